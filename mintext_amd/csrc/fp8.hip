// Blockwise fp8 (OCP e4m3fn) grouped GEMM for the MoE layer on gfx950.
//
// The reference has no fp8 grouped GEMM (its only fp8 code is per-tensor scaling of a dense
// Linear, bzantium/mintext mintext/modules/linear.py:37-57).  Format used here (DeepSeek-V3
// style blockwise scaling):
//   activations  x ~ xq * xs : xq [M,K] e4m3fn, xs [M,K/128] f32 (1x128 groups per row)
//   weights      W ~ wq * ws : wq [E,N,K] e4m3fn (k-contiguous, the per-expert nn.Linear
//                              layout), ws [E,N/128,K/128] f32 (128x128 blocks)
//   scale = amax / 448 (1 when amax == 0), q = RNE(x / scale) saturating at +-448.
//   out[r,n] = sum_kb xs[r,kb] * ws[e,n/128,kb] * sum_{k in kb} xq[r,k] * wq[e,n,k]
// with f32 accumulation (MFMA v_mfma_f32_32x32x64_f8f6f4, scales applied per 128-K block in
// f32 on the partial sums) and a bf16 output, or -- for the gate_up GEMM -- the SwiGLU and
// a 1x128 re-quantisation of its output fused into the epilogue.
#include "common.h"
#include "lds_dma.h"
#include "fp8_tile.h"
#include <type_traits>
#include <utility>

namespace mtx {

struct MTileF8 {
  int e, r0, r1, pad;
};

namespace f8 {

typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int BK = 128;  // bytes of k per step == one scale block

__device__ __forceinline__ int lds_off(int r, int c) { return r * 128 + ((c ^ (r & 7) ^ ((r >> 3) & 7)) << 4); }

// ---- quantisers ------------------------------------------------------------------------------
// 16 elements per lane: a 128-group spans 8 lanes, a wave quantises 8 groups per step, and each
// lane issues the loads of UNR steps before their math so that UNR x 16-32 bytes are in flight
// per lane; the group maximum is a butterfly within the 8 lanes.  Codes go out as one 16-byte
// store per lane.
// P2: power-of-two scales (p2_scale), the codes of x * 2^-e (exact quotients).
template <typename T, int UNR, bool P2 = false>
__global__ __launch_bounds__(256) void quant_rows_kernel(const T* __restrict__ x, int64_t M, int64_t D,
                                                         uint8_t* __restrict__ xq, float* __restrict__ xs) {
  constexpr int EPL = 16, LPG = 8, GPW = 8, NLD = EPL * (int)sizeof(T) / 16;  // 16-byte loads per lane
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPG, gl = lane % LPG;
  const int64_t ng = D / 128;
  const int64_t total = M * ng;
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t t0 = wid * GPW; t0 < total; t0 += nw * GPW * UNR) {
    u32x4 raw[UNR][NLD];
    int64_t tt[UNR];
    bool ok[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t t = t0 + (int64_t)u * nw * GPW + sub;
      ok[u] = t < total;
      tt[u] = ok[u] ? t : total - 1;
      const int64_t r = tt[u] / ng, g = tt[u] - r * ng;
      const u32x4* src = (const u32x4*)(x + r * D + g * 128 + gl * EPL);
#pragma unroll
      for (int l = 0; l < NLD; ++l) raw[u][l] = src[l];
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float v[EPL];
#pragma unroll
      for (int l = 0; l < NLD; ++l) {
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[4 * l + i] = __uint_as_float(raw[u][l][i]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[8 * l + 2 * i] = __uint_as_float(raw[u][l][i] << 16);
            v[8 * l + 2 * i + 1] = __uint_as_float(raw[u][l][i] & 0xffff0000u);
          }
        }
      }
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) m = fmaxf(m, fabsf(v[i]));
      static_assert(LPG == 8, "one 128-group per 8 lanes");
      m = max8_lanes(m);  // DPP lane exchanges, no LDS round trip
      float sc = P2 ? p2_scale(m) : m / 448.0f;
      if (sc == 0.0f) sc = 1.0f;
      u32x4 q;
      if constexpr (P2) {
        const float rsc = __builtin_amdgcn_ldexpf(1.0f, 127 - (int)e8m0_of(sc));  // 2^-e, exact
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = e4m3_pack4(v[4 * i] * rsc, v[4 * i + 1] * rsc, v[4 * i + 2] * rsc, v[4 * i + 3] * rsc);
      } else if (__builtin_expect(div_rn_ok(sc), 1)) {
        const float rsc = 1.0f / sc;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = e4m3_pack4(div_rn(v[4 * i], sc, rsc), div_rn(v[4 * i + 1], sc, rsc), div_rn(v[4 * i + 2], sc, rsc),
                            div_rn(v[4 * i + 3], sc, rsc));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = e4m3_pack4(v[4 * i] / sc, v[4 * i + 1] / sc, v[4 * i + 2] / sc, v[4 * i + 3] / sc);
      }
      if (!ok[u]) continue;
      const int64_t r = tt[u] / ng, g = tt[u] - r * ng;
      *(u32x4*)(xq + r * D + g * 128 + gl * EPL) = q;
      if (gl == 0) xs[r * ng + g] = sc;
    }
  }
}

// One workgroup per 128x128 (Kin x Kout) block of one expert: one scale for the block, codes
// written transposed ([E, Kout, Kin], k contiguous) through LDS.
template <typename T, bool P2 = false>
__global__ __launch_bounds__(256) void quant_weights_kernel(const T* __restrict__ w, int64_t Kin, int64_t Kout,
                                                            uint8_t* __restrict__ wq, float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) uint8_t tt[128 * q8::TSTRIDE];
  __shared__ float red[4];
  using S = q8::TileShape<T>;
  const int64_t e = blockIdx.z, k0 = (int64_t)blockIdx.y * 128, n0 = (int64_t)blockIdx.x * 128;
  q8::Tile<T> t;
  t.load(w + (e * Kin + k0) * Kout + n0, Kout, 128);
  float m[S::VE];
  t.col_amax(m);
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < S::VE; ++j) a = fmaxf(a, m[j]);
  const float s = q8::block_scale<P2>(a, red);
  q8::codes_to_lds_t(t, [&](int) { return s; }, tt);
  __syncthreads();
  q8::lds_t_to_global(tt, wq + (e * Kout + n0) * Kin + k0, Kin);
  if (threadIdx.x == 0) ws[(e * (Kout / 128) + blockIdx.x) * (Kin / 128) + blockIdx.y] = s;
}

// ---- tile scheduler (same contract as the bf16 path) ---------------------------------------------
__global__ __launch_bounds__(1024) void build_tiles_f8_kernel(const int32_t* __restrict__ gs, int E, int M, int BM,
                                                              int* __restrict__ count, MTileF8* __restrict__ tiles) {
  __shared__ int wsum[16];
  __shared__ long long wsum64[16];
  __shared__ int s_total[2];
  const int e = threadIdx.x, lane = e & 63, w = e >> 6;
  const int g = (e < E) ? min(max(gs[e], 0), M) : 0;  // rows past M are dropped
  // row offsets in 64 bits: E groups of up to M rows each can sum past 2^31
  long long incl64 = g;
  for (int off = 1; off < 64; off <<= 1) {
    const long long o = __shfl_up(incl64, off);
    if (lane >= off) incl64 += o;
  }
  if (lane == 63) wsum64[w] = incl64;
  __syncthreads();
  if (e == 0) {
    long long run = 0;
    for (int i = 0; i < 16; ++i) { const long long x = wsum64[i]; wsum64[i] = run; run += x; }
    s_total[0] = (int)min(run, (long long)M);
  }
  __syncthreads();
  const long long start = incl64 - g + wsum64[w];
  const int r0 = (int)min(start, (long long)M), r1 = (int)min(start + g, (long long)M);
  const int nt = (r1 - r0 + BM - 1) / BM;
  __syncthreads();
  int incl = nt;
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  if (e == 0) {
    int run = 0;
    for (int i = 0; i < 16; ++i) { const int x = wsum[i]; wsum[i] = run; run += x; }
    s_total[1] = run;
  }
  __syncthreads();
  const int tstart = incl - nt + wsum[w];
  for (int i = 0; i < nt; ++i) {
    MTileF8 t;
    t.e = e;
    t.r0 = r0 + i * BM;
    t.r1 = min(r0 + (i + 1) * BM, r1);
    t.pad = 0;
    tiles[tstart + i] = t;
  }
  const int used = min(s_total[0], M);
  const int ntail = (M - used + BM - 1) / BM;
  for (int z = e; z < ntail; z += blockDim.x) {  // may exceed the block when many rows are unused
    MTileF8 t;
    t.e = -1;
    t.r0 = used + z * BM;
    t.r1 = min(used + (z + 1) * BM, M);
    t.pad = 0;
    tiles[s_total[1] + z] = t;
  }
  if (e == 0) count[0] = s_total[1] + ntail;
  if (e >= 8 && e < 16) count[e] = 0;  // the persistent kernel's per-XCD tile tickets
}

// ---- GEMM --------------------------------------------------------------------------------------
struct Args {
  const uint8_t* xq;
  const float* xs;
  const uint8_t* wq;
  const float* ws;
  uint16_t* out;      // bf16 [M, ldc] (plain) / optional bf16 SwiGLU output
  uint8_t* outq;      // SwiGLU: e4m3 [M, I]
  float* outs;        // SwiGLU: [M, I/128]
  const int* count;
  const MTileF8* tiles;
  int M, K, N, I, ldc;
  // gathered rows (v4 kernel): sorted row r reads row gather[r] / gather_div of xq and xs
  // (clamped to [0, gather_rows)); the dispatch copy of the quantised tokens is never written
  const int32_t* gather;
  int gather_div, gather_rows;
};

enum { EPI_STORE = 0, EPI_SWIGLU_Q = 1 };

template <int ROWS, int NT>
struct RowLoader {  // ROWS rows x 128 bytes, 16-byte chunks
  static constexpr int CPT = ROWS * 8 / NT;
  static_assert((ROWS * 8) % NT == 0, "split");
  u32x4 r[CPT];
  template <typename RowMap>
  __device__ __forceinline__ void load(const uint8_t* __restrict__ src, int64_t ld, RowMap rowmap, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int q = tid + i * NT;
      r[i] = *(const u32x4*)(src + (int64_t)rowmap(q >> 3) * ld + k0 + (q & 7) * 16);
    }
  }
  __device__ __forceinline__ void store(char* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int q = tid + i * NT;
      *(u32x4*)(lds + lds_off(q >> 3, q & 7)) = r[i];
    }
  }
};

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM* WN * 64, 1) void gmm_fp8_kernel(Args p) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(WTN <= 128 && (128 % WTN == 0 || WTN == 128), "wave N-range within one 128-col scale block");
  static_assert(EPI != EPI_SWIGLU_Q || (TN % 2 == 0 && WN == 2 && BN == 256), "SwiGLU layout");
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128, S_BYTES = BM * 4;
  constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];
  __shared__ float red[BM][2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int nn = (EPI == EPI_SWIGLU_Q) ? (p.I / (BN / 2)) : (p.N / BN);
  const int cnt = p.count[0];
  const int total = cnt * nn;
  const int pid = blockIdx.x;
  const int total8 = (total + 7) & ~7;
  if (pid >= total8) return;
  const int lid = (pid & 7) * (total8 >> 3) + (pid >> 3);
  if (lid >= total) return;
  constexpr int GM = 8;
  const int grp = lid / (GM * nn);
  const int first_m = grp * GM;
  const int gsz = min(GM, cnt - first_m);
  const int local = lid - grp * GM * nn;
  const int mt = first_m + local % gsz;
  const int n_tile = local / gsz;
  const MTileF8 t = p.tiles[mt];
  const int e = t.e, r0 = t.r0, r1 = t.r1;
  const int col0 = n_tile * BN;
  if (e < 0) {
    if (EPI == EPI_SWIGLU_Q) {
      const int c0 = n_tile * (BN / 2);
      for (int i = tid; i < BM * (BN / 2); i += NT) {
        const int r = r0 + i / (BN / 2);
        if (r < r1) {
          p.outq[(int64_t)r * p.I + c0 + i % (BN / 2)] = 0;
          if (p.out) p.out[(int64_t)r * p.I + c0 + i % (BN / 2)] = 0;
        }
      }
      for (int i = tid; i < BM; i += NT)
        if (r0 + i < r1) p.outs[(int64_t)(r0 + i) * (p.I / 128) + c0 / 128] = 1.0f;
    } else {
      for (int i = tid; i < BM * BN; i += NT) {
        const int r = r0 + i / BN;
        if (r < r1) p.out[(int64_t)r * p.ldc + col0 + i % BN] = 0;
      }
    }
    return;
  }
  const int I = p.I;
  // weight row (output column n) of tile-local column c
  auto b_row = [=](int c) -> int {
    if (EPI == EPI_SWIGLU_Q) {
      const int w_ = c / WTN, within = c % WTN;
      const int half = within / (WTN / 2), off = within % (WTN / 2);
      return half * I + n_tile * (BN / 2) + w_ * (WTN / 2) + off;
    }
    return col0 + c;
  };
  const int Mlast = p.M - 1;
  auto a_row = [=](int rr) -> int {
    const int g = r0 + rr;
    return g < Mlast ? g : Mlast;
  };
  const int nkb = p.K / BK;
  const uint8_t* wsrc = p.wq + (int64_t)e * p.N * p.K;
  const float* wsc = p.ws + (int64_t)e * (p.N / 128) * nkb;

  RowLoader<BM, NT> la;
  RowLoader<BN, NT> lb;
  float sreg = 0.0f;  // one A-scale per thread (tid < BM)
  auto issue = [&](int kb) {
    la.load(p.xq, p.K, a_row, kb * BK, tid);
    lb.load(wsrc, p.K, b_row, kb * BK, tid);
    if (tid < BM) sreg = p.xs[(int64_t)a_row(tid) * nkb + kb];
  };
  auto stash = [&](char* st) {
    la.store(st, tid);
    lb.store(st + A_BYTES, tid);
    if (tid < BM) ((float*)(st + A_BYTES + B_BYTES))[tid] = sreg;
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // per-j weight-scale block row (constant over k)
  int sb_row[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) sb_row[j] = b_row(wn * WTN + j * 32) / 128;

  issue(0);
  stash(lds);
  __syncthreads();
  const int frow = lane & 31, fhalf = lane >> 5;
  for (int kb = 0; kb < nkb; ++kb) {
    const char* As = lds + (kb & 1) * STAGE;
    const char* Bs = As + A_BYTES;
    const float* Ss = (const float*)(As + A_BYTES + B_BYTES);
    const bool more = kb + 1 < nkb;
    if (more) issue(kb + 1);
    float sbv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) sbv[j] = wsc[(int64_t)sb_row[j] * nkb + kb];
    f32x16 part[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) part[i][j][v] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      i32x8 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 32 + frow;
        const u32x4 lo = *(const u32x4*)(As + lds_off(r, kk * 4 + fhalf * 2));
        const u32x4 hi = *(const u32x4*)(As + lds_off(r, kk * 4 + fhalf * 2 + 1));
        a[i] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WTN + j * 32 + frow;
        const u32x4 lo = *(const u32x4*)(Bs + lds_off(r, kk * 4 + fhalf * 2));
        const u32x4 hi = *(const u32x4*)(Bs + lds_off(r, kk * 4 + fhalf * 2 + 1));
        b[j] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          part[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i], b[j], part[i][j], 0, 0, 0, 127, 0, 127);
    }
    // promote: acc += part * xs[row] * ws[col block]
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 sa = *(const f32x4*)(Ss + wm * WTM + i * 32 + 8 * q + 4 * fhalf);
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int u = 0; u < 4; ++u) acc[i][j][4 * q + u] = fmaf(part[i][j][4 * q + u], sa[u] * sbv[j], acc[i][j][4 * q + u]);
      }
    }
    if (more) stash(lds + ((kb + 1) & 1) * STAGE);
    __syncthreads();
  }

  const int ccol = lane & 31, rhalf = fhalf * 4;
  if (EPI == EPI_STORE) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = r0 + wm * WTM + i * 32 + 8 * (v >> 2) + rhalf + (v & 3);
          if (row < r1) p.out[(int64_t)row * p.ldc + col0 + wn * WTN + j * 32 + ccol] = f32_to_bf16(acc[i][j][v]);
        }
    return;
  }
  // SwiGLU + 1x128 quantisation: this tile holds y columns [n_tile*128, n_tile*128+128);
  // wave wn holds 64 of them (j < TN/2 gate blocks, paired with up blocks j + TN/2).
  float y[TM][TN / 2][16];
  float rmax[TM][16];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < TN / 2; ++j) {
        const float yy = silu_f32(acc[i][j][v]) * acc[i][j + TN / 2][v];
        y[i][j][v] = yy;
        m = fmaxf(m, fabsf(yy));
      }
      // reduce over the 32 lanes that share this row (lane bits 0..4)
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
      rmax[i][v] = m;
    }
  if (ccol == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[wm * WTM + i * 32 + 8 * (v >> 2) + rhalf + (v & 3)][wn] = rmax[i][v];
  }
  __syncthreads();
  const int ycol0 = n_tile * 128 + wn * 64;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int rl = wm * WTM + i * 32 + 8 * (v >> 2) + rhalf + (v & 3);
      const int row = r0 + rl;
      float s = fmaxf(red[rl][0], red[rl][1]) / 448.0f;
      if (s == 0.0f) s = 1.0f;
      if (row < r1) {
#pragma unroll
        for (int j = 0; j < TN / 2; ++j) {
          const int col = ycol0 + j * 32 + ccol;
          p.outq[(int64_t)row * p.I + col] = f32_to_e4m3(y[i][j][v] / s);
          if (p.out) p.out[(int64_t)row * p.I + col] = f32_to_bf16(y[i][j][v]);
        }
        if (wn == 0 && ccol == 0) p.outs[(int64_t)row * (p.I / 128) + n_tile] = s;
      }
    }
}


// ---- v3: direct-to-LDS ring (256x256 tiles, 8 waves) ---------------------------------------------
// Both operands are k-contiguous, so a ring stage holds 64 k-bytes of 256 x-rows and of 256
// weight rows (32 KB), loaded with global_load_lds_dwordx4 three stages ahead; 16-byte chunk c
// of row r sits at chunk c ^ ((r>>2)&3), which keeps the 32-byte fragment reads conflict-free.
// One v_mfma_scale_f32_32x32x64_f8f6f4 per 32x32 block and stage, operands swapped so that each
// lane owns four consecutive output columns.  Block scales: the accumulators are kept in units of
// the current 128-k block's scale s = xs[row,kb] * ws[nblk,kb]; between blocks they are multiplied
// by s_kb / s_kb+1 (one multiply per accumulator per 128 k, no second accumulator set), and by the
// last block's scale at the end, which gives sum_kb s_kb * P_kb.  The tile's scales are staged in
// LDS once.  Scales must be finite and nonzero (the quantisers never produce 0).
namespace v3 {
constexpr int BM = 256, BN = 256, BKB = 64, NSTAGE = 4, PD = 3;
constexpr int A_BYTES = BM * BKB, B_BYTES = BN * BKB, STAGE = A_BYTES + B_BYTES;
constexpr int MAX_KB = 24;  // K <= 3072
__device__ __forceinline__ int a_off(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }
}  // namespace v3

typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;

template <int EPI>
__global__ __launch_bounds__(512, 2) void gmm_fp8_v3_kernel(Args p) {
  using namespace v3;
  constexpr int WN = 4, NT = 512, WTM = 128, WTN = 64, TM = 4, TN = 2;
  constexpr int A_INSTR = 2, B_INSTR = 2, LPS = A_INSTR + B_INSTR;
  __shared__ __attribute__((aligned(1024))) char lds[NSTAGE * STAGE];
  __shared__ float s_sa[MAX_KB * BM];  // [kb][tile row]
  __shared__ float s_sb[2 * MAX_KB];   // [weight-row half][kb]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int nn = (EPI == EPI_SWIGLU_Q) ? (p.I / 128) : (p.N / BN);
  const int cnt = p.count[0];
  const int total = cnt * nn;
  const int pid = blockIdx.x;
  const int total8 = (total + 7) & ~7;
  if (pid >= total8) return;
  const int lid = (pid & 7) * (total8 >> 3) + (pid >> 3);
  if (lid >= total) return;
  constexpr int GM = 8;
  const int grp = lid / (GM * nn);
  const int first_m = grp * GM;
  const int gsz = min(GM, cnt - first_m);
  const int local = lid - grp * GM * nn;
  const int mt = first_m + local % gsz;
  const int n_tile = local / gsz;
  const MTileF8 t = p.tiles[mt];
  const int e = t.e, r0 = t.r0, r1 = t.r1;
  const int col0 = n_tile * BN;
  if (e < 0) {  // rows past sum(group_sizes)
    if (EPI == EPI_SWIGLU_Q) {
      const int c0 = n_tile * 128;
      for (int i = tid; i < BM * 128; i += NT) {
        const int r = r0 + i / 128;
        if (r < r1) {
          p.outq[(int64_t)r * p.I + c0 + i % 128] = 0;
          if (p.out) p.out[(int64_t)r * p.I + c0 + i % 128] = 0;
        }
      }
      for (int i = tid; i < BM; i += NT)
        if (r0 + i < r1) p.outs[(int64_t)(r0 + i) * (p.I / 128) + n_tile] = 1.0f;
    } else {
      for (int i = tid; i < BM * BN; i += NT) {
        const int r = r0 + i / BN;
        if (r < r1) p.out[(int64_t)r * p.ldc + col0 + i % BN] = 0;
      }
    }
    return;
  }
  const int nkb = p.K / 128, nk = p.K / BKB;
  // weight row of tile-local column c: the SwiGLU tile pairs gate rows n_tile*128 + [0,128)
  // with up rows I + n_tile*128 + [0,128), 32 of each per wave
  auto b_row = [&](int c) -> int {
    if (EPI == EPI_SWIGLU_Q) {
      const int w_ = c / WTN, within = c % WTN;
      return (within / 32) * p.I + n_tile * 128 + w_ * 32 + within % 32;
    }
    return col0 + c;
  };

  // ---- scales of this tile -> LDS (before the ring loads, so their waits stay separate) ----
  {
    const float* wsc = p.ws + (int64_t)e * (p.N / 128) * nkb;
    for (int i = tid; i < BM * nkb; i += NT) {
      const int kb = i / BM, r = i % BM;
      const int gr = min(r0 + r, r1 - 1);
      s_sa[kb * BM + r] = p.xs[(int64_t)gr * nkb + kb];
    }
    if (tid < 2 * nkb) {
      const int h = tid / nkb, kb = tid % nkb;
      const int nblk = (EPI == EPI_SWIGLU_Q) ? (h * (p.I / 128) + n_tile) : (col0 / 128 + h);
      s_sb[h * MAX_KB + kb] = wsc[(int64_t)nblk * nkb + kb];
    }
  }

  // ---- per-lane global sources: lane l of segment s fills row 16s + l/4, chunk slot l%4 ----
  const uint8_t* Bb = p.wq + (int64_t)e * p.N * p.K;
  uint32_t aoff[A_INSTR], boff[B_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int seg = wave * A_INSTR + i;
    const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
    const int gr = min(r0 + r, r1 - 1);  // rows past the group repeat its last row (unused)
    aoff[i] = (uint32_t)gr * (uint32_t)p.K + (uint32_t)(c * 16);
  }
#pragma unroll
  for (int i = 0; i < B_INSTR; ++i) {
    const int seg = wave * B_INSTR + i;
    const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
    boff[i] = (uint32_t)b_row(r) * (uint32_t)p.K + (uint32_t)(c * 16);
  }
  const uint32_t lds_base = lds_addr(lds);
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  // Stages past the end re-read the last one (in bounds) into a ring slot that is no longer
  // read, which keeps the loop body free of branches.
  auto issue_stage = [&](int kt) {
    const uint32_t st = lds_base + (uint32_t)((kt & (NSTAGE - 1)) * STAGE);
    const uint32_t kofs = (uint32_t)min(kt, nk - 1) * BKB;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) gload_lds16(p.xq + aoff[i] + kofs, st + (wave_u * A_INSTR + i) * 1024u);
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i)
      gload_lds16(Bb + boff[i] + kofs, st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
  };

  // ---- fragments: lane l holds row l%32, k bytes 32*(l/32) .. +31 of the stage ------------
  i32x8 fa[2][TM], fb[2][TN];
  const int frow = lane & 31, fhalf = lane >> 5;
  auto ld32 = [&](const char* base, int r) -> i32x8 {
    const u32x4 lo = *(const u32x4*)(base + a_off(r, 2 * fhalf));
    const u32x4 hi = *(const u32x4*)(base + a_off(r, 2 * fhalf + 1));
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  auto read_frags = [&](int kt, int buf, int nb) {
    const char* st = lds + (kt & (NSTAGE - 1)) * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      if (i < nb) fa[buf][i] = ld32(st, wm * WTM + i * 32 + frow);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[buf][j] = ld32(st + A_BYTES, wn * WTN + j * 32 + frow);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // weight-scale half of accumulator column block j
  auto half_of = [&](int j) -> int { return (EPI == EPI_SWIGLU_Q) ? j : (wn >> 1); };
  // the two factors of an accumulator's scale in block kb (never multiplied together, so that two
  // small scales cannot underflow)
  auto sa_of = [&](int i, int kb) -> float { return s_sa[kb * BM + wm * WTM + i * 32 + frow]; };
  auto sb_of = [&](int j, int kb) -> float { return s_sb[half_of(j) * MAX_KB + kb]; };

  // 32-row blocks of this wave that hold rows of the group
  const int nbi = min(max((r1 - r0 - wm * WTM + 31) / 32, 0), TM);

#pragma unroll
  for (int s = 0; s < PD; ++s)
    if (nk > s) issue_stage(s);
  if (nk >= PD) __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
  else __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));
  __syncthreads();  // stages 0 and 1 and the scales are visible
  read_frags(0, 0, nbi);

  // One iteration per 128-k scale block: ring stages 2kb (fragment buffer 0) and 2kb+1
  // (buffer 1), so every fragment index is a compile-time constant.
  auto main_loop = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    const int nb = FULL ? TM : nbi;
    auto mfmas = [&](int buf) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (!FULL && i >= nb) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[buf][j], fa[buf][i], acc[i][j], 0, 0, 0, 127,
                                                                      0, 127);
      }
    };
    auto finish_stage = [&]() {
      // stage kt+2 must have landed before the barrier makes it visible to every wave (stage
      // kt+3, possibly a re-read past the end, may still be in flight)
      __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
      __syncthreads();
    };
    for (int kb = 0; kb < nkb; ++kb) {
      const int kt = 2 * kb;
      const bool more = kb + 1 < nkb;
      // scale factors s_kb / s_kb+1 (read now, applied after this block's MFMAs)
      float f[TM][TN];
      if (more) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            f[i][j] = (sa_of(i, kb) * __builtin_amdgcn_rcpf(sa_of(i, kb + 1))) *
                      (sb_of(j, kb) * __builtin_amdgcn_rcpf(sb_of(j, kb + 1)));
      }
      issue_stage(kt + PD);
      read_frags(kt + 1, 1, nb);
      mfmas(0);
      finish_stage();
      issue_stage(kt + 1 + PD);
      read_frags(kt + 2, 0, nb);  // the last step reads an unused ring slot (in bounds)
      mfmas(1);
      if (more) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (!FULL && i >= nb) continue;
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] *= f[i][j];
        }
      }
      finish_stage();
    }
  };
  if (nbi == TM) main_loop(std::integral_constant<bool, true>());
  else main_loop(std::integral_constant<bool, false>());
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));  // no ring load may land after the workgroup ends

  // ---- epilogue: acc[i][j][4g+q] of lane l is C[row i*32 + l%32][col j*32 + 8g + 4(l/32) + q]
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const float fa = sa_of(i, nkb - 1), fb_ = sb_of(j, nkb - 1);
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = (acc[i][j][v] * fa) * fb_;
    }
  const int erow = wm * WTM + frow;
  if (EPI == EPI_STORE) {
    const int ecol = col0 + wn * WTN + 4 * fhalf;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = r0 + erow + i * 32;
      if (row < r1) {
        uint16_t* orow = p.out + (int64_t)row * p.ldc + ecol;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(bf16x4*)(orow + j * 32 + 8 * g) = bf16x4{(__bf16)acc[i][j][4 * g], (__bf16)acc[i][j][4 * g + 1],
                                                       (__bf16)acc[i][j][4 * g + 2], (__bf16)acc[i][j][4 * g + 3]};
      }
    }
    return;
  }
  // SwiGLU (gate block j = 0, up block j = 1) and 1x128 re-quantisation: the tile holds output
  // columns [n_tile*128, +128), wave wn columns wn*32 + [0,32); the row maximum is combined
  // over the two lanes of a row and over the four waves through LDS (the ring is free now).
  float y[TM][16];
  float* red = (float*)lds;  // [256 rows][4 waves]
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    float m = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      y[i][v] = acc[i][0][v] * acc[i][1][v] * __builtin_amdgcn_rcpf(1.0f + __expf(-acc[i][0][v]));
      m = fmaxf(m, fabsf(y[i][v]));
    }
    m = fmaxf(m, __shfl_xor(m, 32));
    if (fhalf == 0) red[(erow + i * 32) * 4 + wn] = m;
  }
  __syncthreads();
  const int ycol = n_tile * 128 + wn * 32 + 4 * fhalf;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int rl = erow + i * 32, row = r0 + rl;
    const f32x4 mx = *(const f32x4*)(red + rl * 4);
    float sc = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])) / 448.0f;
    if (sc == 0.0f) sc = 1.0f;
    if (row < r1) {
      uint8_t* qrow = p.outq + (int64_t)row * p.I + ycol;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t q = (uint32_t)f32_to_e4m3(y[i][4 * g] / sc) | ((uint32_t)f32_to_e4m3(y[i][4 * g + 1] / sc) << 8) |
                           ((uint32_t)f32_to_e4m3(y[i][4 * g + 2] / sc) << 16) |
                           ((uint32_t)f32_to_e4m3(y[i][4 * g + 3] / sc) << 24);
        *(uint32_t*)(qrow + 8 * g) = q;
      }
      if (p.out) {
        uint16_t* brow = p.out + (int64_t)row * p.I + ycol;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(bf16x4*)(brow + 8 * g) = bf16x4{(__bf16)y[i][4 * g], (__bf16)y[i][4 * g + 1], (__bf16)y[i][4 * g + 2],
                                            (__bf16)y[i][4 * g + 3]};
      }
      if (wn == 0 && fhalf == 0) p.outs[(int64_t)row * (p.I / 128) + n_tile] = sc;
    }
  }
}


// ---- v4: persistent workgroups, block scales streamed through the ring -------------------------
// Same tile, fragments and accumulation as v3, but (1) each workgroup walks a list of tiles and
// the ring keeps loading across tile boundaries (the next tile's first stages are in flight
// while the current tile finishes and stores), and (2) the scales travel with the data: the
// even stage of every 128-k block also carries that block's 256 x-row scales (global_load_lds
// of 4 bytes per lane, waves 0-3) and its two weight-block scales (wave 4), so no tile prologue
// waits on memory.  Needs K >= 256 (four stages per tile, three in flight).
// P2 (power-of-two scales, p2_scale): the scales are E8M0 codes (their f32 exponent fields) given
// to v_mfma_scale_f32_32x32x64_f8f6f4, which multiplies each lane's codes by 2^(code - 127) -- the
// row's 1x128 activation scale and the weight block's 128x128 scale, constant over the MFMA's 64
// k -- so the accumulators stay in true units over all of K: no rescale at the block boundaries
// and no scale multiply in the epilogue.  On the C4 shapes this is 8-9 % faster than the one-wave-
// per-SIMD per-tile kernel it replaced (the same bits: the same MFMA sequence per output element).
namespace v4 {
constexpr int BM = 256, BN = 256, BKB = 64, NSTAGE = 4, PD = 3;
constexpr int A_BYTES = BM * BKB, B_BYTES = BN * BKB;
constexpr int S_OFF = A_BYTES + B_BYTES;  // per slot: [0,1K) x-row scales, [1K,1K+8) weight scales
constexpr int STAGE = S_OFF + 2048;
// m-tiles per scheduling group (consecutive tiles sweep GM m-tiles, then n): 2 for the SwiGLU
// tiles, 8 for the plain-store ones (C4 gate_up with 2 against 8: pow2 -1.5 to -3.3 %, amax -1 to
// +0.2 % over four runs on two boxes; the store tiles -- C4 down, the C5 dlhs -- lose 1.5-3 % with
// 2 or 4)
template <int EPI>
constexpr int gm_of() { return EPI == EPI_SWIGLU_Q ? 2 : 8; }
struct Tile {
  int e, r0, r1, n_tile, zero;
};
}  // namespace v4

template <int EPI, bool P2 = false>
__global__ __launch_bounds__(512, 2) void gmm_fp8_v4_kernel(Args p) {
  using namespace v4;
  using v3::a_off;
  constexpr int WN = 4, WTM = 128, WTN = 64, TM = 4, TN = 2;
  constexpr int LPS = 4;  // data loads per wave and stage; even stages add one scale load
  __shared__ __attribute__((aligned(1024))) char lds[NSTAGE * STAGE];
  __shared__ float red[BM * 4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const int wm = wave / WN, wn = wave % WN;
  const int nn = (EPI == EPI_SWIGLU_Q) ? (p.I / 128) : (p.N / BN);
  const int cnt = p.count[0];
  const int total = cnt * nn;
  // XCD x (= blockIdx % 8) sweeps tiles [x*per, (x+1)*per) with its gridDim/8 workgroups
  const int nx = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), q = (int)(blockIdx.x >> 3);
  const int per = (total + 7) >> 3;
  const int lid_end = min((xcd + 1) * per, total);
  int lid = xcd * per + q;
  if (lid >= lid_end) return;
  const int nkb = p.K / 128, nk = p.K / BKB;

  auto decode = [&](int l) -> Tile {
    constexpr int GM = gm_of<EPI>();
    const int grp = l / (GM * nn);
    const int first_m = grp * GM;
    const int gsz = min(GM, cnt - first_m);
    const int local = l - grp * GM * nn;
    // the tile list is read-only here: read through the scalar cache (constant address space,
    // uniform index), so that the tile switch waits on lgkmcnt, not on the ring's vmcnt
    typedef const __attribute__((address_space(4))) int cint_t;
    const int ti = __builtin_amdgcn_readfirstlane(first_m + local % gsz);
    const cint_t* tp = (const cint_t*)(uintptr_t)(p.tiles + ti);
    MTileF8 t;
    t.e = tp[0];
    t.r0 = tp[1];
    t.r1 = tp[2];
    Tile T;
    T.zero = t.e < 0;
    T.e = t.e < 0 ? 0 : t.e;  // rows past sum(group_sizes): computed with expert 0, stored as 0
    T.r0 = t.r0;
    T.r1 = t.r1;
    T.n_tile = local / gsz;
    return T;
  };
  // weight row of tile-local column c (SwiGLU tiles pair gate and up rows, 32 of each per wave)
  auto b_row = [&](const Tile& T, int c) -> int {
    if (EPI == EPI_SWIGLU_Q) {
      const int w_ = c / WTN, within = c % WTN;
      return (within / 32) * p.I + T.n_tile * 128 + w_ * 32 + within % 32;
    }
    return T.n_tile * BN + c;
  };
  struct Src {
    uint32_t aoff[2], boff[2];
    const uint8_t* B;
    const float* sb;  // this wave's scale base (uniform) ...
    uint32_t so;      // ... + this lane's byte offset: its scale for k-block 0 (one float per block after it)
  };
  // row of xq / xs that holds sorted row r (the row itself unless the rows are gathered)
  auto x_row = [&](int r) -> int {
    return p.gather ? min(max(p.gather[r], 0) / p.gather_div, p.gather_rows - 1) : r;
  };
  auto make_src = [&](const Tile& T) -> Src {
    Src S;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int seg = wave * 2 + i;
      const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
      S.aoff[i] = (uint32_t)x_row(min(T.r0 + r, T.r1 - 1)) * (uint32_t)p.K + (uint32_t)(c * 16);
      S.boff[i] = (uint32_t)b_row(T, r) * (uint32_t)p.K + (uint32_t)(c * 16);
    }
    S.B = p.wq + (int64_t)T.e * p.N * p.K;
    if (wave_u < 4) {
      S.sb = p.xs;
      S.so = (uint32_t)x_row(min(T.r0 + 64 * wave + lane, T.r1 - 1)) * (uint32_t)nkb * 4u;
    } else if (wave_u == 4) {
      const int h = lane & 1;
      const int nblk = (EPI == EPI_SWIGLU_Q) ? (h * (p.I / 128) + T.n_tile) : (T.n_tile * 2 + h);
      S.sb = p.ws + (int64_t)T.e * (p.N / 128) * nkb;
      S.so = (uint32_t)nblk * (uint32_t)nkb * 4u;
    } else {
      S.sb = p.xs;  // filler load, keeps the per-wave load count uniform
      S.so = (uint32_t)x_row(T.r0) * (uint32_t)nkb * 4u;
    }
    return S;
  };

  Tile cur = decode(lid);
  int lid_next = lid + nx;
  Tile nxt = lid_next < lid_end ? decode(lid_next) : cur;
  Src scur = make_src(cur), snxt = make_src(nxt);
  // Tiles past each workgroup's first two come from its XCD's ticket counter (count[8 + xcd],
  // zeroed by the tile-list kernel): ticket t is tile xcd*per + 2*nx + t, so a workgroup that
  // finishes early takes more tiles.  Wave 0 takes the ticket of the tile after next at the start
  // of each epilogue and publishes it through LDS before the epilogue's last barrier (by then the
  // ring loads issued before the epilogue have landed, so its wait for the atomic costs little);
  // inside the k-loop the ticket's register would not fit beside the accumulators.
#ifndef MTX_F8_TICKETS
#define MTX_F8_TICKETS 1
#endif
  __shared__ int s_ticket;
  const uint32_t lds_base = lds_addr(lds);
  // issue ring step g = stage kt of the current tile, or of the next one when kt >= nk
  // (uniform bases in SGPRs, per-lane 32-bit offsets)
  auto issue = [&](int g, int kt, bool even) {
    const bool in = kt < nk;
    const int k = in ? kt : kt - nk;
    const uint32_t st = lds_base + (uint32_t)((g & (NSTAGE - 1)) * STAGE);
    const uint32_t kofs = (uint32_t)k * BKB;
    const uint8_t* A = p.xq + kofs;
#pragma unroll
    for (int i = 0; i < 2; ++i) gload_lds16_s(A, in ? scur.aoff[i] : snxt.aoff[i], st + (wave_u * 2 + i) * 1024u);
    const uint8_t* B = (in ? scur.B : snxt.B) + kofs;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      gload_lds16_s(B, in ? scur.boff[i] : snxt.boff[i], st + (uint32_t)A_BYTES + (wave_u * 2 + i) * 1024u);
    if (even) gload_lds4_s((in ? scur.sb : snxt.sb) + (k >> 1), in ? scur.so : snxt.so, st + (uint32_t)S_OFF + wave_u * 256u);
  };

  const int frow = lane & 31, fhalf = lane >> 5;
  auto ld32 = [&](const char* base, int r) -> i32x8 {
    const u32x4 lo = *(const u32x4*)(base + a_off(r, 2 * fhalf));
    const u32x4 hi = *(const u32x4*)(base + a_off(r, 2 * fhalf + 1));
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  // Rotating fragments: one A set fr_a[TM] and two B sets fr_b[2][TN].  During a stage the
  // A fragment of row block i is reloaded from the next stage right after its last MFMA, and
  // the next stage's B fragments go to the other B set, so the live fragments fit beside the
  // 128 accumulators without serialising every LDS read before its MFMA.
  i32x8 fr_a[TM], fr_b[2][TN];
  auto rd_a = [&](int g_, int i) -> i32x8 {
    return ld32(lds + (g_ & (NSTAGE - 1)) * STAGE, wm * WTM + i * 32 + frow);
  };
  auto rd_b = [&](int g_, int j) -> i32x8 {
    return ld32(lds + (g_ & (NSTAGE - 1)) * STAGE + A_BYTES, wn * WTN + j * 32 + frow);
  };
  // scales of the k-block whose even stage sits in ring step g.  Weight-block scales: SwiGLU
  // tiles use both (gate columns j = 0, up columns j = 1); a plain tile's wave uses only the
  // block holding its 64 columns, read once into sb[0] so that every index stays static.
  constexpr int NSB = (EPI == EPI_SWIGLU_Q) ? 2 : 1;
  float sa_c[TM], sb_c[NSB], sa_n[TM], sb_n[NSB];
  auto read_scales = [&](int g, float* sa, float* sb) {
    const float* sc = (const float*)(lds + (g & (NSTAGE - 1)) * STAGE + S_OFF);
#pragma unroll
    for (int i = 0; i < TM; ++i) sa[i] = sc[wm * WTM + i * 32 + frow];
    if (EPI == EPI_SWIGLU_Q) {
      sb[0] = sc[256];
      sb[NSB - 1] = sc[257];
    } else {
      sb[0] = sc[256 + (wn >> 1)];
    }
  };
  auto half_of = [&](int j) -> int { return (EPI == EPI_SWIGLU_Q) ? j : 0; };
  // P2 (power-of-two scales): the same block scales as E8M0 codes for the MFMA's scale operands --
  // the lane's four row-block codes packed one per byte (opsel i), the weight block code(s) per half
  uint32_t ea_c = 0, ea_n = 0, eb_c[NSB] = {}, eb_n[NSB] = {};
  auto read_codes = [&](int g, uint32_t& ea, uint32_t (&eb)[NSB]) {
    const float* sc = (const float*)(lds + (g & (NSTAGE - 1)) * STAGE + S_OFF);
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) s |= e8m0_of(sc[wm * WTM + i * 32 + frow]) << (8 * i);
    ea = s;
    if (EPI == EPI_SWIGLU_Q) {
      eb[0] = e8m0_of(sc[256]);
      eb[NSB - 1] = e8m0_of(sc[257]);
    } else {
      eb[0] = e8m0_of(sc[256 + (wn >> 1)]);
    }
  };
  // acc += B_j A_i with the codes of the current block (opsel must be a constant: one case per i)
  auto mfma_p2 = [&](const i32x8& b, const i32x8& a, const f32x16& c, int i, uint32_t eb) -> f32x16 {
    switch (i) {
      case 0: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb, 0, (int)ea_c);
      case 1: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb, 1, (int)ea_c);
      case 2: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb, 2, (int)ea_c);
      default: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb, 3, (int)ea_c);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // prologue: ring steps 0..2; steps 0 and 1 landed (step 2 = LPS + 1 loads may be in flight)
  issue(0, 0, true);
  issue(1, 1, false);
  issue(2, 2, true);
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS + 1));
  __syncthreads();
  if constexpr (P2) read_codes(0, ea_c, eb_c);
  else read_scales(0, sa_c, sb_c);
#pragma unroll
  for (int i = 0; i < TM; ++i) fr_a[i] = rd_a(0, i);
#pragma unroll
  for (int j = 0; j < TN; ++j) fr_b[0][j] = rd_b(0, j);
  int g = 0;

  // One stage of the rotating schedule: MFMAs of ring step g_ on fr_a / fr_b[cb], with the
  // fragments of step g_+1 read in between; at a k-block boundary each accumulator moves from
  // the previous block's scale units to this block's (f = s_prev / s_this) before its MFMA.
  auto rot_stage = [&](int g_, int cb, bool rescale, const float (&f)[TM][NSB]) {
#pragma unroll
    for (int j = 0; j < TN; ++j) fr_b[cb ^ 1][j] = rd_b(g_ + 1, j);
    // accumulator q = i*TN + j is rescaled (block boundary only) one slot ahead of its MFMA,
    // while the previous MFMA runs, so that no MFMA waits on the multiplies of its own input
    auto rescale_acc = [&](int q) {
      const int i = q / TN, j = q % TN;
      const float fj = f[i][half_of(j)];
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] *= fj;
    };
    if (rescale) rescale_acc(0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (P2)
          acc[i][j] = mfma_p2(fr_b[cb][j], fr_a[i], acc[i][j], i, eb_c[half_of(j)]);
        else
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr_b[cb][j], fr_a[i], acc[i][j], 0, 0, 0, 127,
                                                                      0, 127);
        if (rescale && i * TN + j + 1 < TM * TN) rescale_acc(i * TN + j + 1);
      }
      fr_a[i] = rd_a(g_ + 1, i);
    }
  };

  // One 128-k block (an even and an odd stage); FIRST: the tile's first block (no rescale).
  auto kblock = [&](int kb, auto first_tag) {
    constexpr bool FIRST = decltype(first_tag)::value;
    const int kt = 2 * kb;
    // even stage kt (ring step g): B fragments in set 0
    issue(g + PD, kt + PD, false);
    float f[TM][NSB] = {};
    if (FIRST) {
      rot_stage(g, 0, false, f);
    } else if (P2) {  // true units throughout: only the codes change
      ea_c = ea_n;
#pragma unroll
      for (int h = 0; h < NSB; ++h) eb_c[h] = eb_n[h];
      rot_stage(g, 0, false, f);
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < NSB; ++h)  // (sa_c / sa_n) * (sb_c / sb_n): no product of two small scales
          f[i][h] = (sa_c[i] * __builtin_amdgcn_rcpf(sa_n[i])) * (sb_c[h] * __builtin_amdgcn_rcpf(sb_n[h]));
#pragma unroll
      for (int i = 0; i < TM; ++i) sa_c[i] = sa_n[i];
#pragma unroll
      for (int h = 0; h < NSB; ++h) sb_c[h] = sb_n[h];
      rot_stage(g, 0, true, f);
    }
    // Step g+2 landed (g+3 may be in flight), then a bare s_barrier: __syncthreads() would
    // also wait for this wave's outstanding LDS reads, which are the fragments of the next
    // step (visible since the previous barrier) and need not complete before it.  Slots are
    // refilled only after every wave's MFMAs consumed the fragments read from them.
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS));
    __builtin_amdgcn_s_barrier();
    // odd stage kt+1 (ring step g+1): B fragments in set 1
    issue(g + 1 + PD, kt + 1 + PD, true);
    if constexpr (P2) read_codes(g + 2, ea_n, eb_n);  // next block's codes (or the next tile's)
    else read_scales(g + 2, sa_n, sb_n);              // next block's scales (or the next tile's)
    rot_stage(g + 1, 1, false, f);
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS + 1));  // step g+3 landed (g+4 may be in flight)
    __builtin_amdgcn_s_barrier();
    g += 2;
  };

  for (;;) {
    kblock(0, std::true_type());
    for (int kb = 1; kb < nkb; ++kb) kblock(kb, std::false_type());

    int tk = 0;
    if (MTX_F8_TICKETS && wave_u == 0 && lane == 0) {
      // the per-lane form (no wave-level rewrite, so no vmcnt(0) at the draw) where it measured
      // faster: the amax store mode (C4 down -1.7 %; the other modes -0.5 to +7 %)
      if constexpr (EPI == EPI_STORE && !P2)
        tk = lane_fetch_add(const_cast<int*>(p.count) + 8 + xcd, 1);
      else
        tk = __hip_atomic_fetch_add(const_cast<int*>(p.count) + 8 + xcd, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // ---- epilogue of the current tile (the next tile's first stages are in flight) ---------
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const float fa = sa_c[i], fb_ = sb_c[half_of(j)];
#pragma unroll
        for (int v = 0; v < 16; ++v)  // (not 0 * x: x may be NaN)
          acc[i][j][v] = cur.zero ? 0.0f : (P2 ? acc[i][j][v] : (acc[i][j][v] * fa) * fb_);
      }
    // Outputs are staged through ring slot g-1 (the tile's last stage, consumed; the next DMA
    // into it is issued after the closing barrier) so that every global store writes 16
    // contiguous bytes per lane and whole 128-byte lines per group of 8 lanes (32 KB used).
    // The bare barriers of the k-loop do not order LDS reads (the compiler may place a stage's
    // last fragment reads and their waits after them), so every wave's reads complete before
    // the staging writes: an LDS-only release fence, then a barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    char* stg = lds + ((g - 1) & (NSTAGE - 1)) * STAGE;
    const int erow = wm * WTM + frow;
    if (EPI == EPI_STORE) {
      // per wave: 32 rows x 64 bf16 columns (128 bytes) at a time; 16-byte chunk c of row r is
      // stored at chunk c ^ (r & 7)
      char* wst = stg + wave * 4096;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
            *(bf16x4*)(wst + frow * 128 + (((4 * j + gq) ^ (frow & 7)) << 4) + 8 * fhalf) =
                bf16x4{(__bf16)acc[i][j][4 * gq], (__bf16)acc[i][j][4 * gq + 1], (__bf16)acc[i][j][4 * gq + 2],
                       (__bf16)acc[i][j][4 * gq + 3]};
        __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int rloc = rr * 8 + (lane >> 3);
          const u32x4 v = *(const u32x4*)(wst + rloc * 128 + (((lane & 7) ^ (rloc & 7)) << 4));
          const int row = cur.r0 + wm * WTM + i * 32 + rloc;
          if (row < cur.r1)
            *(u32x4*)(p.out + (int64_t)row * p.ldc + cur.n_tile * BN + wn * WTN + (lane & 7) * 8) = v;
        }
        __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);  // reads done before the next block overwrites
      }
      if (MTX_F8_TICKETS && wave_u == 0 && lane == 0) s_ticket = tk;
      __syncthreads();  // staging slot free before the next tile's first ring load
    } else {
      float y[TM][16];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        float m = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          y[i][v] = acc[i][0][v] * acc[i][1][v] * __builtin_amdgcn_rcpf(1.0f + __expf(-acc[i][0][v]));
          m = fmaxf(m, fabsf(y[i][v]));
        }
        m = fmaxf(m, __shfl_xor(m, 32));
        if (fhalf == 0) red[(erow + i * 32) * 4 + wn] = m;
      }
      __syncthreads();
      // e4m3 codes of the tile's 128 output columns: [256 rows][128 bytes], 16-byte chunk c of
      // row r at chunk c ^ (r & 7)
      const int ycol = wn * 32 + 4 * fhalf;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int rl = erow + i * 32, row = cur.r0 + rl;
        const f32x4 mx = *(const f32x4*)(red + rl * 4);
        const float amax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
        float sc, inv;
        if constexpr (P2) {
          sc = p2_scale(amax);
          inv = __builtin_amdgcn_ldexpf(1.0f, 127 - (int)e8m0_of(sc));  // 2^-e, exact
        } else {
          sc = amax / 448.0f;
          if (sc == 0.0f) sc = 1.0f;
          inv = 1.0f / sc;
        }
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const uint32_t qv = e4m3_pack4(y[i][4 * gq] * inv, y[i][4 * gq + 1] * inv, y[i][4 * gq + 2] * inv,
                                         y[i][4 * gq + 3] * inv);
          const int cb = ycol + 8 * gq;
          *(uint32_t*)(stg + rl * 128 + (((cb >> 4) ^ (rl & 7)) << 4) + (cb & 15)) = qv;
        }
        if (row < cur.r1) {
          if (p.out) {
            uint16_t* brow = p.out + (int64_t)row * p.I + cur.n_tile * 128 + ycol;
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
              *(bf16x4*)(brow + 8 * gq) = bf16x4{(__bf16)y[i][4 * gq], (__bf16)y[i][4 * gq + 1],
                                                 (__bf16)y[i][4 * gq + 2], (__bf16)y[i][4 * gq + 3]};
          }
          if (wn == 0 && fhalf == 0) p.outs[(int64_t)row * (p.I / 128) + cur.n_tile] = sc;
        }
      }
      if (MTX_F8_TICKETS && wave_u == 0 && lane == 0) s_ticket = tk;
      __syncthreads();
      // 256 rows x 128 bytes: 8 lanes per row, 8 rows per wave instruction
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int rl = wave * 32 + rr * 8 + (lane >> 3);
        const u32x4 v = *(const u32x4*)(stg + rl * 128 + (((lane & 7) ^ (rl & 7)) << 4));
        const int row = cur.r0 + rl;
        if (row < cur.r1) *(u32x4*)(p.outq + (int64_t)row * p.I + cur.n_tile * 128 + (lane & 7) * 16) = v;
      }
      __syncthreads();  // red and the staging slot are reused by the next tile
    }
    // the tile after next (s_ticket is rewritten only in the next tile's epilogue)
    const int lid_after = MTX_F8_TICKETS ? xcd * per + 2 * nx + s_ticket : lid_next + nx;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // ---- next tile ------------------------------------------------------------------------
    lid = lid_next;
    if (lid >= lid_end) break;
    cur = nxt;
    scur = snxt;
    lid_next = lid_after;
    if (lid_next < lid_end) {
      nxt = decode(lid_next);
      snxt = make_src(nxt);
    }
    if constexpr (P2) {
      ea_c = ea_n;
#pragma unroll
      for (int h = 0; h < NSB; ++h) eb_c[h] = eb_n[h];
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i) sa_c[i] = sa_n[i];
#pragma unroll
      for (int h = 0; h < NSB; ++h) sb_c[h] = sb_n[h];
    }
  }
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));  // filler loads of the last steps land before exit
}

}  // namespace f8

static inline int64_t f8_ws_bytes(int64_t M, int64_t E, int64_t BM) {
  return 256 + (ceil_div(M, BM) + E + 1) * (int64_t)sizeof(MTileF8);
}

// Power-of-two scales (p2): the persistent kernel with the block scales as the MFMA's E8M0
// operands; it needs K >= 256 and 32-bit operand offsets (MTX_ERR_UNSUPPORTED otherwise).
template <int EPI>
static int launch_fp8_v4_p2(const f8::Args& a, const int32_t* gs, int64_t E, int64_t nn, void* ws, hipStream_t st) {
  const int64_t a_rows = a.gather ? a.gather_rows : a.M;
  const bool off32 = a_rows * a.K < (int64_t(1) << 32) && (int64_t)a.N * a.K < (int64_t(1) << 32);
  if (!(off32 && a.K >= 256)) return MTX_ERR_UNSUPPORTED;
  int* count = (int*)ws;
  MTileF8* tiles = (MTileF8*)((char*)ws + 256);
  hipLaunchKernelGGL(f8::build_tiles_f8_kernel, dim3(1), dim3(1024), 0, st, gs, (int)E, a.M, 256, count, tiles);
  f8::Args b = a;
  b.count = count;
  b.tiles = tiles;
  int64_t grid = round_up((ceil_div(a.M, 256) + E + 1) * nn, 8);
  const int ncu = device_cu_count();
  const int64_t cap = ncu > 0 ? round_up(ncu, 8) : 256;
  if (grid > cap) grid = cap;  // persistent: one workgroup per CU (a multiple of the 8 XCDs)
  hipLaunchKernelGGL((f8::gmm_fp8_v4_kernel<EPI, true>), dim3((unsigned)grid), dim3(512), 0, st, b);
  return check_launch();
}

template <int EPI>
static int launch_fp8(const f8::Args& a, const int32_t* gs, int64_t E, int64_t nn, void* ws, hipStream_t st) {
  const int64_t a_rows = a.gather ? a.gather_rows : a.M;
  const bool off32 = a_rows * a.K < (int64_t(1) << 32) && (int64_t)a.N * a.K < (int64_t(1) << 32);
  if (a.gather && !(off32 && a.K >= 256)) return MTX_ERR_UNSUPPORTED;  // gathered rows: v4 kernel only
  if (off32 && a.K >= 256) {
    int* count = (int*)ws;
    MTileF8* tiles = (MTileF8*)((char*)ws + 256);
    hipLaunchKernelGGL(f8::build_tiles_f8_kernel, dim3(1), dim3(1024), 0, st, gs, (int)E, a.M, 256, count, tiles);
    f8::Args b = a;
    b.count = count;
    b.tiles = tiles;
    int64_t grid = round_up((ceil_div(a.M, 256) + E + 1) * nn, 8);
    const int ncu = device_cu_count();
    const int64_t cap = ncu > 0 ? round_up(ncu, 8) : 256;
    if (grid > cap) grid = cap;  // persistent: one workgroup per CU (a multiple of the 8 XCDs)
    hipLaunchKernelGGL((f8::gmm_fp8_v4_kernel<EPI>), dim3((unsigned)grid), dim3(512), 0, st, b);
    return check_launch();
  }
  const bool v3ok = a.K <= 128 * f8::v3::MAX_KB && off32;
  if (v3ok) {
    int* count = (int*)ws;
    MTileF8* tiles = (MTileF8*)((char*)ws + 256);
    hipLaunchKernelGGL(f8::build_tiles_f8_kernel, dim3(1), dim3(1024), 0, st, gs, (int)E, a.M, 256, count, tiles);
    f8::Args b = a;
    b.count = count;
    b.tiles = tiles;
    const int64_t grid = round_up((ceil_div(a.M, 256) + E + 1) * nn, 8);
    hipLaunchKernelGGL((f8::gmm_fp8_v3_kernel<EPI>), dim3((unsigned)grid), dim3(512), 0, st, b);
    return check_launch();
  }
  constexpr int BM = 128, BN = 256;
  int* count = (int*)ws;
  MTileF8* tiles = (MTileF8*)((char*)ws + 256);
  hipLaunchKernelGGL(f8::build_tiles_f8_kernel, dim3(1), dim3(1024), 0, st, gs, (int)E, a.M, BM, count, tiles);
  f8::Args b = a;
  b.count = count;
  b.tiles = tiles;
  const int64_t grid = round_up((ceil_div(a.M, BM) + E + 1) * nn, 8);
  hipLaunchKernelGGL((f8::gmm_fp8_kernel<BM, BN, 2, 2, EPI>), dim3((unsigned)grid), dim3(256), 0, st, b);
  return check_launch();
}

}  // namespace mtx

using namespace mtx;

template <bool P2>
static int quant_rows_entry(const void* x, int dtype, int64_t M, int64_t D, uint8_t* xq, float* x_scale,
                            void* stream) {
  if (M < 0 || D < 0 || D % 128 != 0 || (dtype != MTX_F32 && dtype != MTX_BF16)) return MTX_ERR_ARG;
  if (M == 0 || D == 0) return MTX_OK;
  if (!x || !xq || !x_scale) return MTX_ERR_ARG;
  if (((uintptr_t)x % 16) || ((uintptr_t)xq % 16)) return MTX_ERR_ARG;
  constexpr int UNR = 4;
  int64_t blocks = ceil_div(M * (D / 128), (int64_t)8 * 4 * UNR);  // 8 groups per wave and step, 4 waves
  if (blocks > 16384) blocks = 16384;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MTX_F32)
    hipLaunchKernelGGL((f8::quant_rows_kernel<float, UNR, P2>), dim3(blocks), dim3(256), 0, st, (const float*)x, M,
                       D, xq, x_scale);
  else
    hipLaunchKernelGGL((f8::quant_rows_kernel<uint16_t, UNR, P2>), dim3(blocks), dim3(256), 0, st,
                       (const uint16_t*)x, M, D, xq, x_scale);
  return check_launch();
}

extern "C" int mtx_quant_fp8_rows(const void* x, int dtype, int64_t M, int64_t D, uint8_t* xq, float* x_scale,
                                  void* stream) {
  return quant_rows_entry<false>(x, dtype, M, D, xq, x_scale, stream);
}

extern "C" int mtx_quant_fp8_rows_p2(const void* x, int dtype, int64_t M, int64_t D, uint8_t* xq, float* x_scale,
                                     void* stream) {
  return quant_rows_entry<true>(x, dtype, M, D, xq, x_scale, stream);
}

template <bool P2>
static int quant_weights_entry(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout, uint8_t* w_q,
                               float* w_scale, void* stream) {
  if (E < 0 || Kin < 0 || Kout < 0 || Kin % 128 || Kout % 128 || (dtype != MTX_F32 && dtype != MTX_BF16))
    return MTX_ERR_ARG;
  if (E == 0 || Kin == 0 || Kout == 0) return MTX_OK;
  if (!w || !w_q || !w_scale) return MTX_ERR_ARG;
  if (((uintptr_t)w | (uintptr_t)w_q) % 16) return MTX_ERR_ARG;  // 16-byte loads and stores
  if (E > 65535 || Kin / 128 > 65535) return MTX_ERR_UNSUPPORTED;
  dim3 grid((unsigned)(Kout / 128), (unsigned)(Kin / 128), (unsigned)E);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MTX_F32)
    hipLaunchKernelGGL((f8::quant_weights_kernel<float, P2>), grid, dim3(256), 0, st, (const float*)w, Kin, Kout,
                       w_q, w_scale);
  else
    hipLaunchKernelGGL((f8::quant_weights_kernel<uint16_t, P2>), grid, dim3(256), 0, st, (const uint16_t*)w, Kin,
                       Kout, w_q, w_scale);
  return check_launch();
}

extern "C" int mtx_quant_fp8_weights(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout, uint8_t* w_q,
                                     float* w_scale, void* stream) {
  return quant_weights_entry<false>(w, dtype, E, Kin, Kout, w_q, w_scale, stream);
}

extern "C" int mtx_quant_fp8_weights_p2(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout,
                                        uint8_t* w_q, float* w_scale, void* stream) {
  return quant_weights_entry<true>(w, dtype, E, Kin, Kout, w_q, w_scale, stream);
}

static int fp8_checks(const void* xq, const float* xs, const uint8_t* wq, const float* ws, const int32_t* gs,
                      int64_t M, int64_t Kin, int64_t E, void* workspace, int64_t workspace_bytes) {
  if (M < 0 || M > INT32_MAX / 2 || E < 1 || E > 1024 || Kin <= 0 || Kin % 128) return MTX_ERR_ARG;
  if (!workspace || workspace_bytes < f8_ws_bytes(M, E, 64)) return MTX_ERR_WORKSPACE;
  if (M > 0 && (!xq || !xs || !wq || !ws || !gs)) return MTX_ERR_ARG;
  if (((uintptr_t)xq | (uintptr_t)wq) % 16) return MTX_ERR_ARG;
  return MTX_OK;
}

static int gmm_fp8_entry(bool p2, const uint8_t* xq, const float* x_scale, const uint8_t* w_q, const float* w_scale,
                         const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* out,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = fp8_checks(xq, x_scale, w_q, w_scale, group_sizes, M, Kin, E, workspace, workspace_bytes);
  if (rc) return rc;
  if (Kout <= 0 || Kout % 256) return (Kout % 128 == 0 && Kout > 0) ? MTX_ERR_UNSUPPORTED : MTX_ERR_ARG;
  if (M == 0) return MTX_OK;
  if (!out) return MTX_ERR_ARG;
  f8::Args a{};
  a.xq = xq;
  a.xs = x_scale;
  a.wq = w_q;
  a.ws = w_scale;
  a.out = (uint16_t*)out;
  a.M = (int)M;
  a.K = (int)Kin;
  a.N = (int)Kout;
  a.I = 0;
  a.ldc = (int)Kout;
  if (p2) return launch_fp8_v4_p2<f8::EPI_STORE>(a, group_sizes, E, Kout / 256, workspace, (hipStream_t)stream);
  return launch_fp8<f8::EPI_STORE>(a, group_sizes, E, Kout / 256, workspace, (hipStream_t)stream);
}

extern "C" int mtx_gmm_fp8(const uint8_t* xq, const float* x_scale, const uint8_t* w_q, const float* w_scale,
                           const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* out,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  return gmm_fp8_entry(false, xq, x_scale, w_q, w_scale, group_sizes, M, Kin, Kout, E, out, workspace,
                       workspace_bytes, stream);
}

extern "C" int mtx_gmm_fp8_p2(const uint8_t* xq, const float* x_scale, const uint8_t* w_q, const float* w_scale,
                              const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* out,
                              void* workspace, int64_t workspace_bytes, void* stream) {
  return gmm_fp8_entry(true, xq, x_scale, w_q, w_scale, group_sizes, M, Kin, Kout, E, out, workspace,
                       workspace_bytes, stream);
}

static int fp8_swiglu_entry(const uint8_t* xq, const float* x_scale, const uint8_t* w_q, const float* w_scale,
                            const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t I, int64_t E, uint8_t* out_q,
                            float* out_scale, void* out_bf16, void* workspace, int64_t workspace_bytes, void* stream,
                            const int32_t* gather, int64_t gather_div, int64_t gather_rows, bool p2 = false) {
  int rc = fp8_checks(xq, x_scale, w_q, w_scale, group_sizes, M, Kin, E, workspace, workspace_bytes);
  if (rc) return rc;
  if (I <= 0 || I % 128) return MTX_ERR_ARG;
  if (gather && (gather_div < 1 || gather_div > INT32_MAX || gather_rows < 0 || gather_rows > INT32_MAX / 2 ||
                 (gather_rows == 0 && M > 0)))
    return MTX_ERR_ARG;
  if (M == 0) return MTX_OK;
  if (!out_q || !out_scale) return MTX_ERR_ARG;
  f8::Args a{};
  a.gather = gather;
  a.gather_div = (int)gather_div;
  a.gather_rows = (int)gather_rows;
  a.xq = xq;
  a.xs = x_scale;
  a.wq = w_q;
  a.ws = w_scale;
  a.out = (uint16_t*)out_bf16;
  a.outq = out_q;
  a.outs = out_scale;
  a.M = (int)M;
  a.K = (int)Kin;
  a.N = (int)(2 * I);
  a.I = (int)I;
  a.ldc = (int)I;
  if (p2) return launch_fp8_v4_p2<f8::EPI_SWIGLU_Q>(a, group_sizes, E, I / 128, workspace, (hipStream_t)stream);
  return launch_fp8<f8::EPI_SWIGLU_Q>(a, group_sizes, E, I / 128, workspace, (hipStream_t)stream);
}

extern "C" int mtx_gmm_fp8_swiglu(const uint8_t* xq, const float* x_scale, const uint8_t* w_q, const float* w_scale,
                                  const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t I, int64_t E,
                                  uint8_t* out_q, float* out_scale, void* out_bf16, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  return fp8_swiglu_entry(xq, x_scale, w_q, w_scale, group_sizes, M, Kin, I, E, out_q, out_scale, out_bf16, workspace,
                          workspace_bytes, stream, nullptr, 1, 0);
}

extern "C" int mtx_gmm_fp8_swiglu_gathered(const uint8_t* xq, const float* x_scale, int64_t x_rows,
                                           const int32_t* row_index, int64_t index_div, const uint8_t* w_q,
                                           const float* w_scale, const int32_t* group_sizes, int64_t M, int64_t Kin,
                                           int64_t I, int64_t E, uint8_t* out_q, float* out_scale, void* out_bf16,
                                           void* workspace, int64_t workspace_bytes, void* stream) {
  if (!row_index && M > 0) return MTX_ERR_ARG;
  return fp8_swiglu_entry(xq, x_scale, w_q, w_scale, group_sizes, M, Kin, I, E, out_q, out_scale, out_bf16, workspace,
                          workspace_bytes, stream, row_index, index_div, x_rows);
}

extern "C" int mtx_gmm_fp8_swiglu_p2(const uint8_t* xq, const float* x_scale, const uint8_t* w_q,
                                     const float* w_scale, const int32_t* group_sizes, int64_t M, int64_t Kin,
                                     int64_t I, int64_t E, uint8_t* out_q, float* out_scale, void* out_bf16,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  return fp8_swiglu_entry(xq, x_scale, w_q, w_scale, group_sizes, M, Kin, I, E, out_q, out_scale, out_bf16, workspace,
                          workspace_bytes, stream, nullptr, 1, 0, true);
}

extern "C" int mtx_gmm_fp8_swiglu_gathered_p2(const uint8_t* xq, const float* x_scale, int64_t x_rows,
                                              const int32_t* row_index, int64_t index_div, const uint8_t* w_q,
                                              const float* w_scale, const int32_t* group_sizes, int64_t M,
                                              int64_t Kin, int64_t I, int64_t E, uint8_t* out_q, float* out_scale,
                                              void* out_bf16, void* workspace, int64_t workspace_bytes,
                                              void* stream) {
  if (!row_index && M > 0) return MTX_ERR_ARG;
  return fp8_swiglu_entry(xq, x_scale, w_q, w_scale, group_sizes, M, Kin, I, E, out_q, out_scale, out_bf16, workspace,
                          workspace_bytes, stream, row_index, index_div, x_rows, true);
}
