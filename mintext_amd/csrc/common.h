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
  // one branch per four values (the clamp turns NaN into -448; NaN is rare)
  if (__builtin_expect((a != a) | (b != b) | (c != c) | (d != d), 0)) {
    const float v[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (v[i] != v[i]) q = (q & ~(0xffu << (8 * i))) | ((uint32_t)(f32_to_e4m3(v[i])) << (8 * i));
  }
  return q;
}

// Lane exchange of step S of an all-reduce over aligned groups of 2^(S+1) lanes.  Steps 0 and 1
// are xor 1 and xor 2 (DPP quad permutes); steps 2 and 3 pair the two halves of each 8- and
// 16-lane group by mirroring (DPP row_half_mirror, row_mirror), which after steps 0..S-1 hands
// every lane the same partial as the xor-4 / xor-8 partner would; step 4 is xor 16 (ds_swizzle,
// bitmask mode) and step 5 xor 32.  So the results equal an xor butterfly's bit for bit (the
// combines are commutative), without the LDS round trip of ds_bpermute.
template <int S>
__device__ __forceinline__ int lane_xchg(int v) {
  if constexpr (S == 0) return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);
  else if constexpr (S == 1) return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);
  else if constexpr (S == 2) return __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false);
  else if constexpr (S == 3) return __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false);
  else if constexpr (S == 4) return __builtin_amdgcn_ds_swizzle(v, 0x401F);
  else return __shfl_xor(v, 32);
}
template <int S>
__device__ __forceinline__ float lane_xchg(float v) {
  return __int_as_float(lane_xchg<S>(__float_as_int(v)));
}
// maximum over each aligned group of 8 lanes (every lane gets it)
__device__ __forceinline__ float max8_lanes(float m) {
  m = fmaxf(m, lane_xchg<0>(m));
  m = fmaxf(m, lane_xchg<1>(m));
  return fmaxf(m, lane_xchg<2>(m));
}

// Division by a quantisation scale b shared by a group of values, in four VALU instructions
// instead of the ten of the full IEEE division: with rb = 1.0f / b (correctly rounded) and
// q = RN(a * rb), RN(q + (a - b*q) * rb) is RN(a / b), the residual a - b*q being exact in one
// FMA (Markstein's correction, IBM J. Res. Develop. 34(1), 1990).  Valid for b in
// [2^-64, 2^100] (div_rn_ok): the result is the IEEE quotient bit for bit whenever |a| >= 2^-100
// or a == 0, and the quotient has a's sign (copysign, for a == -0).  Smaller nonzero |a| can put
// the residual in the subnormal range and the quotient one ulp off, but such quotients are below
// 2^-36 and their e4m3 code (+-0) is the same.  Callers take the IEEE division when
// div_rn_ok(b) fails.
__device__ __forceinline__ bool div_rn_ok(float b) { return b >= 0x1p-64f && b <= 0x1p100f; }
__device__ __forceinline__ float div_rn(float a, float b, float rb) {
  const float q = a * rb;
  return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q, b, a), rb, q), a);
}

// Power-of-two quantisation scale (the MFMA block-scale mode): the smallest 2^e, e in [-126, 127],
// with amax / 2^e <= 448 -- e = ceil(log2(amax / 448)) for normal amax, written on the bits:
// amax = 1.f x 2^(E-127) is at most 448 x 2^e = 1.75 x 2^(8+e) iff e >= E - 135 (+1 when f > 0.75).
// 1 when amax == 0 (as the amax / 448 mode); an infinite or NaN amax gives 2^120 or 2^121.  The
// quotient x / 2^e is then x * 2^-e exactly, and the MFMA's E8M0 scale operand is e + 127, the
// f32 exponent field of the scale.
__device__ __forceinline__ float p2_scale(float amax) {
  if (amax == 0.0f) return 1.0f;
  const uint32_t u = __float_as_uint(amax);
  int e = (int)((u >> 23) & 0xFFu) - 135 + ((u & 0x7FFFFFu) > 0x600000u ? 1 : 0);
  e = e < -126 ? -126 : (e > 127 ? 127 : e);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}
// E8M0 code (biased exponent) of a power-of-two scale in [2^-126, 2^127]
__device__ __forceinline__ uint32_t e8m0_of(float s) { return (__float_as_uint(s) >> 23) & 0xFFu; }

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

// Eight consecutive elements p[i .. i+7] as floats and back (i a multiple of 8, p 16-byte
// aligned): one or two 16-byte accesses, the same conversions as the scalar helpers above.
typedef __attribute__((ext_vector_type(4))) unsigned int v4u32;
__device__ __forceinline__ void ld8(const float* p, int64_t i, float v[8]) {
  const v4u32 a = *(const v4u32*)(p + i), b = *(const v4u32*)(p + i + 4);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[q] = __uint_as_float(a[q]);
    v[4 + q] = __uint_as_float(b[q]);
  }
}
__device__ __forceinline__ void ld8(const uint16_t* p, int64_t i, float v[8]) {
  const v4u32 a = *(const v4u32*)(p + i);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = __uint_as_float(a[q] << 16);
    v[2 * q + 1] = __uint_as_float(a[q] & 0xffff0000u);
  }
}
__device__ __forceinline__ void st8(float* p, int64_t i, const float v[8]) {
  v4u32 a, b;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = __float_as_uint(v[q]);
    b[q] = __float_as_uint(v[4 + q]);
  }
  *(v4u32*)(p + i) = a;
  *(v4u32*)(p + i + 4) = b;
}
__device__ __forceinline__ void st8(uint16_t* p, int64_t i, const float v[8]) {
  v4u32 a;
#pragma unroll
  for (int q = 0; q < 4; ++q) a[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
  *(v4u32*)(p + i) = a;
}
// A relaxed agent-scope fetch-add issued by one lane whose result is first needed much later (a
// persistent kernel's tile ticket, read at the end of the epilogue).  The address goes through a
// VGPR so that the compiler does not rewrite it into a wave-level atomic, whose result it reads
// back at once behind a full vmcnt wait -- that wait would also drain the next tile's ring loads.
__device__ __forceinline__ int lane_fetch_add(int* p, int v) {
  typedef __attribute__((address_space(1))) int gint;  // a global atomic, not a flat one
  uintptr_t a = (uintptr_t)p;
  asm volatile("" : "+v"(a));
  return __hip_atomic_fetch_add((gint*)a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Non-temporal loads (data read once: streamed past the caches), same conversions as ld8.
__device__ __forceinline__ void ld8_nt(const float* p, int64_t i, float v[8]) {
  const v4u32 a = __builtin_nontemporal_load((const v4u32*)(p + i));
  const v4u32 b = __builtin_nontemporal_load((const v4u32*)(p + i + 4));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[q] = __uint_as_float(a[q]);
    v[4 + q] = __uint_as_float(b[q]);
  }
}
__device__ __forceinline__ void ld8_nt(const uint16_t* p, int64_t i, float v[8]) {
  const v4u32 a = __builtin_nontemporal_load((const v4u32*)(p + i));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = __uint_as_float(a[q] << 16);
    v[2 * q + 1] = __uint_as_float(a[q] & 0xffff0000u);
  }
}
// Non-temporal stores (data written once and not read soon: streamed past the caches).
__device__ __forceinline__ void st8_nt(uint16_t* p, int64_t i, const float v[8]) {
  v4u32 a;
#pragma unroll
  for (int q = 0; q < 4; ++q) a[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
  __builtin_nontemporal_store(a, (v4u32*)(p + i));
}
__device__ __forceinline__ void st8_nt(float* p, int64_t i, const float v[8]) {
  v4u32 a, b;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = __float_as_uint(v[q]);
    b[q] = __float_as_uint(v[4 + q]);
  }
  __builtin_nontemporal_store(a, (v4u32*)(p + i));
  __builtin_nontemporal_store(b, (v4u32*)(p + i + 4));
}

}  // namespace mtx
