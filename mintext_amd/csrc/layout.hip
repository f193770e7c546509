// Expert weight layouts on gfx950: batched transpose-copy between HF's per-expert [out, in]
// weights and the fused [in, out] layout the grouped GEMMs read (bzantium/mintext
// mintext/checkpoint/conversion.py:80-166: _import_expert_weights / _export_expert_weights).
//
// out[b][c][r] = in[b][r][c] for r < R, c < C, with independent batch and row strides on both
// sides, so that one call writes the gate half and one the up half of a fused gate_up tensor
// (column offset = pointer offset, row stride 2I), or reads them back.  Element size 2 or 4
// bytes.  HBM-bound: 2 * B * R * C * elem bytes per call.
//
// A workgroup moves one 64x64 tile: 16-byte coalesced loads of 64 input rows into LDS, then
// 16-byte coalesced stores of 64 output rows read down the LDS columns (rows padded by one
// 16-byte chunk so that the column reads spread over the banks).  Tiles that are ragged or not
// 16-byte aligned take a per-element path.
#include "common.h"

namespace mtx {
namespace lay {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
constexpr int TILE = 64;

// 16 bytes from 8 bf16 / 4 f32 elements
__device__ __forceinline__ u32x4 pack16(const uint16_t (&v)[8]) {
  return u32x4{v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16), v[4] | ((uint32_t)v[5] << 16),
               v[6] | ((uint32_t)v[7] << 16)};
}
__device__ __forceinline__ u32x4 pack16(const float (&v)[4]) {
  return u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
}

template <typename T>
__global__ __launch_bounds__(256) void transpose_batched_kernel(const T* __restrict__ in, int64_t R, int64_t C,
                                                                int64_t in_bs, int64_t in_ld, T* __restrict__ out,
                                                                int64_t out_bs, int64_t out_ld, int64_t tiles_c,
                                                                int vec_ok) {
  constexpr int EPC = 16 / sizeof(T);           // elements per 16-byte chunk
  constexpr int CPR = TILE / EPC;               // chunks per tile row
  constexpr int LD = TILE + EPC;                // padded LDS row (elements)
  __shared__ __attribute__((aligned(16))) T tile[TILE * LD];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * TILE, c0 = (int64_t)(blockIdx.x % tiles_c) * TILE;
  const T* src = in + b * in_bs;
  T* dst = out + b * out_bs;
  const bool full = vec_ok && r0 + TILE <= R && c0 + TILE <= C;
  if (full) {
    for (int q = threadIdx.x; q < TILE * CPR; q += blockDim.x) {
      const int r = q / CPR, ch = q % CPR;
      const u32x4 v = *(const u32x4*)(src + (r0 + r) * in_ld + c0 + ch * EPC);
      *(u32x4*)(tile + r * LD + ch * EPC) = v;
    }
    __syncthreads();
    for (int q = threadIdx.x; q < TILE * CPR; q += blockDim.x) {
      const int c = q / CPR, ch = q % CPR;  // output row c (input column), chunk of input rows
      T v[EPC];
#pragma unroll
      for (int e = 0; e < EPC; ++e) v[e] = tile[(ch * EPC + e) * LD + c];
      *(u32x4*)(dst + (c0 + c) * out_ld + r0 + ch * EPC) = pack16(v);
    }
  } else {
    for (int q = threadIdx.x; q < TILE * TILE; q += blockDim.x) {
      const int r = q / TILE, c = q % TILE;
      if (r0 + r < R && c0 + c < C) tile[r * LD + c] = src[(r0 + r) * in_ld + c0 + c];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < TILE * TILE; q += blockDim.x) {
      const int c = q / TILE, r = q % TILE;
      if (r0 + r < R && c0 + c < C) dst[(c0 + c) * out_ld + r0 + r] = tile[r * LD + c];
    }
  }
}

}  // namespace lay
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_transpose_batched(const void* in, int dtype, int64_t B, int64_t R, int64_t C, int64_t in_batch_stride,
                                     int64_t in_ld, void* out, int64_t out_batch_stride, int64_t out_ld,
                                     void* stream) {
  if (dtype != MTX_F32 && dtype != MTX_BF16) return MTX_ERR_ARG;
  if (B < 0 || R < 0 || C < 0) return MTX_ERR_ARG;
  if (B == 0 || R == 0 || C == 0) return MTX_OK;
  if (!in || !out || in_ld < C || out_ld < R) return MTX_ERR_ARG;
  if (B > 65535 || ceil_div(R, lay::TILE) > 65535) return MTX_ERR_ARG;
  const int64_t es = dtype == MTX_F32 ? 4 : 2;
  const int64_t epc = 16 / es;
  const bool vec_ok = ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0) && in_ld % epc == 0 &&
                      out_ld % epc == 0 && in_batch_stride % epc == 0 && out_batch_stride % epc == 0;
  const int64_t tiles_c = ceil_div(C, lay::TILE);
  if (tiles_c > INT32_MAX) return MTX_ERR_ARG;
  dim3 grid((unsigned)tiles_c, (unsigned)ceil_div(R, lay::TILE), (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MTX_F32)
    hipLaunchKernelGGL(lay::transpose_batched_kernel<float>, grid, dim3(256), 0, st, (const float*)in, R, C,
                       in_batch_stride, in_ld, (float*)out, out_batch_stride, out_ld, tiles_c, vec_ok ? 1 : 0);
  else
    hipLaunchKernelGGL(lay::transpose_batched_kernel<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)in, R, C,
                       in_batch_stride, in_ld, (uint16_t*)out, out_batch_stride, out_ld, tiles_c, vec_ok ? 1 : 0);
  return check_launch();
}
