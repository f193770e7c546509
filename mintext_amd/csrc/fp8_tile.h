// Quantisation of one 128 x 128 tile of a row-major bf16/f32 matrix to e4m3fn codes, shared by the
// weight prepacks and the grouped transposing quantiser (gfx950, 256 threads per workgroup).
//
// Loads: 16 bytes per lane (8 bf16 or 4 f32 of one row), a row spread over 16 (bf16) or 32 (f32)
// lanes, every load of the tile issued before any math.  Thread (column group cl, row slot rl)
// holds rows 4 (rl + TR h) + q (q = 0..3), so that it owns four consecutive rows of each of its
// columns and can pack their four codes into one 32-bit word for the transposed layout.
// Scales are amax / 448 (1 when the amax is 0) or the power-of-two p2_scale(amax), over the whole
// tile or per column; codes are e4m3 of value / scale (the IEEE quotient's code, through div_rn;
// exact for a power-of-two scale), by e4m3_pack4.
#pragma once
#include "common.h"

namespace mtx {
namespace q8 {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

template <typename T>
struct TileShape {
  static constexpr int VE = 16 / (int)sizeof(T);  // elements per 16-byte load
  static constexpr int LPR = 128 / VE;            // lanes per row
  static constexpr int TR = 256 / LPR;            // row slots
  static constexpr int G4 = 128 / (4 * TR);       // groups of four rows per thread
  static constexpr int NLD = 4 * G4;              // loads per thread
};

// the tile's values in registers: raw[h][q] = row 4 (rl + TR h) + q, columns cl*VE .. +VE-1;
// rows >= nrows read as zero (no load)
template <typename T>
struct Tile {
  using S = TileShape<T>;
  u32x4 raw[S::G4][4];
  int cl, rl;

  __device__ __forceinline__ void load(const T* __restrict__ src, int64_t ld, int nrows) {
    const int tid = threadIdx.x;
    cl = tid % S::LPR;
    rl = tid / S::LPR;
    const T* p = src + cl * S::VE;
#pragma unroll
    for (int h = 0; h < S::G4; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 4 * (rl + S::TR * h) + q;
        raw[h][q] = r < nrows ? *(const u32x4*)(p + (int64_t)r * ld) : u32x4{0u, 0u, 0u, 0u};
      }
  }
  // element j (column cl*VE + j) of load (h, q) as float
  __device__ __forceinline__ float at(int h, int q, int j) const {
    if constexpr (sizeof(T) == 4) return __uint_as_float(raw[h][q][j]);
    else return __uint_as_float((j & 1) ? (raw[h][q][j >> 1] & 0xffff0000u) : (raw[h][q][j >> 1] << 16));
  }
  // amax of each of this thread's columns over its rows
  __device__ __forceinline__ void col_amax(float (&m)[S::VE]) const {
#pragma unroll
    for (int j = 0; j < S::VE; ++j) {
      float a = 0.0f;
#pragma unroll
      for (int h = 0; h < S::G4; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) a = fmaxf(a, fabsf(at(h, q, j)));
      m[j] = a;
    }
  }
};

// amax / 448 (1 when amax == 0), or with P2 the power-of-two scale p2_scale(amax)
template <bool P2 = false>
__device__ __forceinline__ float scale_of(float amax) {
  if constexpr (P2) return p2_scale(amax);
  float s = amax / 448.0f;
  return s == 0.0f ? 1.0f : s;
}

// one scale for the whole tile (256 threads; red: 4 floats of LDS)
template <bool P2 = false>
__device__ __forceinline__ float block_scale(float m, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  return scale_of<P2>(r);
}

// Codes of the tile transposed into LDS: tt[c * TSTRIDE + r] = code of (row r, column c), written as
// one 32-bit word per (column, group of four rows).  sc(j) is the scale of column cl*VE + j.
constexpr int TSTRIDE = 132;  // bytes per transposed row: 4-byte aligned, 2-way bank spread
template <typename T, typename SC>
__device__ __forceinline__ void codes_to_lds_t(const Tile<T>& t, SC sc, uint8_t* tt) {
  using S = TileShape<T>;
  auto put = [&](auto quot) {
#pragma unroll
    for (int h = 0; h < S::G4; ++h)
#pragma unroll
      for (int j = 0; j < S::VE; ++j) {
        const uint32_t w = e4m3_pack4(quot(t.at(h, 0, j), j), quot(t.at(h, 1, j), j), quot(t.at(h, 2, j), j),
                                      quot(t.at(h, 3, j), j));
        *(uint32_t*)(tt + (t.cl * S::VE + j) * TSTRIDE + 4 * (t.rl + S::TR * h)) = w;
      }
  };
  // one branch per lane: the four-instruction quotient when every scale of the lane's columns
  // allows it, the IEEE division otherwise (the same codes either way)
  bool fast = true;
  float rs[S::VE];
#pragma unroll
  for (int j = 0; j < S::VE; ++j) {
    fast = fast && div_rn_ok(sc(j));
    rs[j] = 1.0f / sc(j);
  }
  if (__builtin_expect(fast, 1)) put([&](float a, int j) { return div_rn(a, sc(j), rs[j]); });
  else put([&](float a, int j) { return a / sc(j); });
}

// 128 transposed rows of 128 bytes from LDS to dst + c * ld (16 bytes per lane, 8 lanes per row)
__device__ __forceinline__ void lds_t_to_global(const uint8_t* tt, uint8_t* __restrict__ dst, int64_t ld) {
  const int tid = threadIdx.x, seg = tid & 7;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int c = p * 32 + (tid >> 3);
    const uint8_t* s = tt + c * TSTRIDE + seg * 16;
    const u32x4 v{*(const uint32_t*)s, *(const uint32_t*)(s + 4), *(const uint32_t*)(s + 8),
                  *(const uint32_t*)(s + 12)};
    *(u32x4*)(dst + (int64_t)c * ld + seg * 16) = v;
  }
}

// Codes of the tile in its own layout: dst + r * ld + column (VE bytes per load, one row of the
// tile is 128 contiguous bytes written by LPR lanes).
template <typename T>
__device__ __forceinline__ void codes_to_global(const Tile<T>& t, float s, uint8_t* __restrict__ dst, int64_t ld) {
  using S = TileShape<T>;
  uint8_t* p = dst + t.cl * S::VE;
  auto put = [&](auto quot) {
#pragma unroll
    for (int h = 0; h < S::G4; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t r = 4 * (t.rl + S::TR * h) + q;
        if constexpr (S::VE == 8) {
          const uint32_t lo =
              e4m3_pack4(quot(t.at(h, q, 0)), quot(t.at(h, q, 1)), quot(t.at(h, q, 2)), quot(t.at(h, q, 3)));
          const uint32_t hi =
              e4m3_pack4(quot(t.at(h, q, 4)), quot(t.at(h, q, 5)), quot(t.at(h, q, 6)), quot(t.at(h, q, 7)));
          *(u32x2*)(p + r * ld) = u32x2{lo, hi};
        } else {
          *(uint32_t*)(p + r * ld) =
              e4m3_pack4(quot(t.at(h, q, 0)), quot(t.at(h, q, 1)), quot(t.at(h, q, 2)), quot(t.at(h, q, 3)));
        }
      }
  };
  const float rs = 1.0f / s;
  if (__builtin_expect(div_rn_ok(s), 1)) put([&](float a) { return div_rn(a, s, rs); });
  else put([&](float a) { return a / s; });
}

}  // namespace q8
}  // namespace mtx
