// Ragged grouped GEMM for the MoE layer on gfx950.
//
// Semantics (bzantium/mintext mintext/kernels/grouped_matmul.py):
//   gmm   : out[r] = x[r] @ W[g(r)], rows grouped contiguously by group_sizes
//           (jax.lax.ragged_dot, grouped_matmul.py:58-76,143-147,242-277); rows past
//           sum(group_sizes) are zero.
//   dlhs  : dx[r] = g[r] @ W[g(r)]^T  (ragged_dot(grad, swapaxes(W,1,2)), :162-176)
//   tgmm  : dW[e] = x[rows_e]^T @ g[rows_e], zeros for an empty group (:197-235)
//   swiglu: silu(h[:, :I]) * h[:, I:]  (mintext/modules/moe.py:195-196), fused into the
//           gate_up GEMM epilogue so h never reaches HBM.
//
// group_sizes stays on the device: a one-workgroup prologue (build_tiles_kernel) turns it
// into a compact list of (expert, row_begin, row_end) M-tiles plus group offsets; the GEMM
// grid is sized to the upper bound ceil(M/BM) + E + 1 tiles and surplus workgroups exit.
//
// bf16 path: CDNA4 MFMA v_mfma_f32_32x32x16_bf16 with f32 accumulation.  The main kernel
// (gmm_v3_kernel, FWD / SWIGLU / DLHS / TGMM) computes 256x256 (or 128x256) output tiles with
// 8 (4) waves; every operand load is a global_load_lds_dwordx4 straight into a 4-deep (3-deep) LDS
// ring, three stages ahead of the MFMAs, with 16-byte chunks XOR-swizzled so that the DMA writes
// and the fragment reads are bank-conflict-free.  Operands whose reduction dim is contiguous in
// HBM are read as fragments with ds_read_b128; the others (W in the forward pass, both operands
// of tgmm) keep their natural layout and are turned into MFMA operands by ds_read_b64_tr_b16
// (gfx950 transpose read).  The epilogue (SwiGLU fused for gate_up) stages the tile through the
// idle ring and writes whole 128-byte lines.  gmm_mfma_kernel, an earlier register-staged design
// (two LDS buffers, 8x8 register transposes), runs only the shapes whose operands exceed 32-bit
// byte offsets.
// f32 path (and shapes the MFMA tiling does not cover): an LDS-tiled exact-fp32 FMA kernel.
#include "common.h"
#include "lds_dma.h"
#include <type_traits>
#include <algorithm>
#include <mutex>

namespace mtx {

// One m-tile of the tile list: expert e (-1: rows past sum(group_sizes), stored as zeros) and rows
// [r0, r1).  pad is 0, or, when the tile builder merges remainder m-tiles into scheduling groups,
// the tile's group: first m-tile of the group << 8 | m-tiles in the group.
struct MTile {
  int e, r0, r1, pad;
};

// ---- tile scheduler ---------------------------------------------------------------------------
// Workspace layout (ints): [0] m-tile count, [1] m-tiles with an expert, [4 .. 11] tickets of the
// per-XCD tile queues (zeroed by the tile-list kernel), [16 .. 16+E] group offsets (E+1, clamped to M),
// [32+E .. ) expert order by descending group size (E), then the MTile array (16B aligned).
struct GmmWs {
  int* count;
  int* offsets;
  int* order;
  MTile* tiles;
  int* split_cnt;     // arrival counters of split tiles (zeroed by build_tiles_kernel)
  float* split_part;  // fp32 partial tiles of split pieces
};
// Split tail (256x256 store tiles, FWD/DLHS).  Workgroup pid is dispatched to XCD pid % 8 and
// each CU holds one 256-row workgroup, so an XCD runs its tiles in rounds of (CUs per XCD).
// When the last round holds at most half as many tiles as CUs (rem <= kSplitMaxRem), those rem
// tiles are split along K into S = min(kSplitMaxS, CUs / rem) pieces, dispatched after the
// whole tiles; each piece stores an f32 partial tile, and the piece that arrives last (per-tile
// counter) sums the partials in piece order and runs the epilogue.  No workgroup waits on
// another, and the sum does not depend on arrival order.  The dispatch assumption only
// affects speed: any placement gives the same result.  At most kSplitItems pieces per XCD.
constexpr int kSplitXcd = 8, kSplitItems = 32, kSplitMaxRem = 16, kSplitMaxS = 4;
constexpr int64_t kSplitSlotFloats = 256 * 256;
static inline int64_t gmm_ws_tiles_off(int64_t E) { return round_up((int64_t)(48 + 2 * E + 1) * 4, 256); }
static inline int64_t gmm_max_tiles(int64_t M, int64_t E, int64_t BM) { return ceil_div(M, BM) + E + 1; }
static inline int64_t gmm_ws_split_off(int64_t M, int64_t E) {
  return round_up(gmm_ws_tiles_off(E) + gmm_max_tiles(M, E, 64) * (int64_t)sizeof(MTile), 256);
}
static inline int64_t gmm_ws_split_bytes() {
  return 1024 + (int64_t)kSplitXcd * kSplitItems * kSplitSlotFloats * 4;
}
static inline GmmWs gmm_ws(void* ws, int64_t M, int64_t E) {
  GmmWs w;
  int* b = (int*)ws;
  w.count = b;
  w.offsets = b + 16;
  w.order = b + 32 + E + 1;
  w.tiles = (MTile*)((char*)ws + gmm_ws_tiles_off(E));
  w.split_cnt = (int*)((char*)ws + gmm_ws_split_off(M, E));
  w.split_part = (float*)((char*)w.split_cnt + 1024);
  return w;
}

// One workgroup of 1024 threads, E <= 1024.
__global__ __launch_bounds__(1024) void build_tiles_kernel(const int32_t* __restrict__ gs, int E, int M, int BM,
                                                           int* __restrict__ count, int* __restrict__ offsets,
                                                           int* __restrict__ order, MTile* __restrict__ tiles,
                                                           int need_order, int* __restrict__ split_cnt, int spread,
                                                           int align, int merge) {
  __shared__ int wsum[16];
  __shared__ long long wsum64[16];
  if (split_cnt && threadIdx.x < kSplitXcd * kSplitMaxRem) split_cnt[threadIdx.x] = 0;
  if (threadIdx.x >= 4 && threadIdx.x < 4 + kSplitXcd) count[threadIdx.x] = 0;  // tile queue tickets
  __shared__ __attribute__((aligned(16))) int s_gs[1024];
  __shared__ int s_total[2];
  const int e = threadIdx.x, lane = e & 63, w = e >> 6;
  const int g = (e < E) ? min(max(gs[e], 0), M) : 0;  // rows past M are dropped
  s_gs[e] = g;
  // exclusive scan of g -> row offsets (64-bit safe: M < 2^31 is checked on the host)
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
  if (e < E) offsets[e] = r0;
  if (e == 0) offsets[E] = min(s_total[0], M);
  __syncthreads();
  // exclusive scan of tile counts
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
  // Tiles are written by all threads, tile j by thread j % 1024: its expert is the last one whose
  // first tile is <= j (experts without tiles share their successor's start), so a skewed
  // expert's tiles do not serialise on one thread.
  __shared__ int s_tstart[1024], s_r0[1024], s_r1[1024];
  if (e < E) {
    s_tstart[e] = incl - nt + wsum[w];
    s_r0[e] = r0;
    s_r1[e] = r1;
  }
  // Spread order (spread > 0, for schedules of one m-tile per group): the m-tiles of experts with
  // at least `spread` tiles (a folded shared expert) go to evenly spaced positions of the list --
  // big tile b at floor((2b+1) N / 2B) of N -- and the other tiles fill the rest in expert order,
  // so that every XCD's contiguous range holds its share of them.
  __shared__ int s_bstart[1024], s_sstart[1024], s_nbig[1];
  // Aligned order (align = G > 1, the scheduling group size): expert e's first floor(nt_e / G) * G
  // m-tiles come first, in expert order, so that every group of G consecutive m-tiles belongs to one
  // expert (its tiles share each weight strip), and the experts' remaining nt_e % G m-tiles follow at
  // the end of the list, in expert order.  s_bstart / s_sstart hold the two sections' starts.
  // merge > 0: an expert with at least one full group and at most `merge` m-tiles past its last
  // group keeps them in that group (a group of G + r), so that they read the expert's weight
  // strips from L2 beside their siblings instead of streaming them again from HBM at the end of
  // the list; every tile then records its group (MTile::pad = first m-tile << 8 | size).
  auto aligned_count = [&](int n) -> int {
    const int a = (n / align) * align;
    return (merge > 0 && a > 0 && n - a <= merge) ? n : a;
  };
  if (align > 1) {
    const int na = (e < E) ? aligned_count(nt) : 0;
    const int nr = (e < E) ? nt - na : 0;
    int ai = na, ri = nr;
    for (int off = 1; off < 64; off <<= 1) {
      const int oa = __shfl_up(ai, off), orr = __shfl_up(ri, off);
      if (lane >= off) {
        ai += oa;
        ri += orr;
      }
    }
    __shared__ int wsa[16], wsr[16];
    if (lane == 63) {
      wsa[w] = ai;
      wsr[w] = ri;
    }
    __syncthreads();
    if (e == 0) {
      int ra = 0, rr = 0;
      for (int i = 0; i < 16; ++i) {
        const int xa = wsa[i], xr = wsr[i];
        wsa[i] = ra;
        wsr[i] = rr;
        ra += xa;
        rr += xr;
      }
      s_nbig[0] = ra;
    }
    __syncthreads();
    if (e < E) {
      s_bstart[e] = ai - na + wsa[w];
      s_sstart[e] = ri - nr + wsr[w];
    }
  }
  if (spread > 0) {
    const int nbig = (e < E && nt >= spread) ? nt : 0;
    int bincl = nbig;
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(bincl, off);
      if (lane >= off) bincl += o;
    }
    __syncthreads();  // wsum is reused
    if (lane == 63) wsum[w] = bincl;
    __syncthreads();
    if (e == 0) {
      int run = 0;
      for (int i = 0; i < 16; ++i) { const int x = wsum[i]; wsum[i] = run; run += x; }
      s_nbig[0] = run;
    }
    __syncthreads();
    if (e < E) {
      s_bstart[e] = bincl - nbig + wsum[w];
      s_sstart[e] = s_tstart[e] - s_bstart[e];  // tiles of the non-big experts before e
    }
  }
  __syncthreads();
  const int ntiles = s_total[1];
  const int nbig_total = (spread > 0) ? s_nbig[0] : 0;
  const int used = min(s_total[0], M);
  const int ntail = (M - used + BM - 1) / BM;
  // group record of list position j past the aligned section: fixed groups of `align` from its end
  auto tail_group = [&](int j) -> int {
    const int na_total = s_nbig[0];
    const int first = na_total + ((j - na_total) / align) * align;
    return (first << 8) | min(align, ntiles + ntail - first);
  };
  for (int j = e; j < ntiles; j += blockDim.x) {
    // position j -> list (start array) and index in it
    const int* starts = s_tstart;
    int idx = j;
    if (nbig_total > 0) {
      const int64_t B = nbig_total, N = ntiles;
      const int64_t num = 2 * B * (j + 1) - N;  // big slots <= j: b with (2b+1) N < 2B (j+1)
      const int cnt = num <= 0 ? 0 : (int)min(B, (num + 2 * N - 1) / (2 * N));
      const bool isbig = cnt > 0 && ((2 * (int64_t)(cnt - 1) + 1) * N) / (2 * B) == j;
      starts = isbig ? s_bstart : s_sstart;
      idx = isbig ? cnt - 1 : j - cnt;
    }
    int first = 0;  // index within the expert of the section's first tile
    if (align > 1) {
      const int na_total = s_nbig[0];
      starts = j < na_total ? s_bstart : s_sstart;
      idx = j < na_total ? j : j - na_total;
    }
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (starts[mid] <= idx) lo = mid;
      else hi = mid - 1;
    }
    const int na_lo = (align > 1) ? aligned_count((s_r1[lo] - s_r0[lo] + BM - 1) / BM) : 0;
    if (align > 1 && j >= s_nbig[0]) first = na_lo;
    const int i = first + idx - starts[lo];
    MTile t;
    t.e = lo;
    t.r0 = s_r0[lo] + i * BM;
    t.r1 = min(s_r0[lo] + (i + 1) * BM, s_r1[lo]);
    t.pad = 0;
    if (align > 1 && merge > 0) {
      if (j < s_nbig[0]) {  // aligned section: the expert's last group takes its merged tiles
        const int ng = na_lo / align, gi = min(i / align, ng - 1);
        t.pad = ((s_bstart[lo] + gi * align) << 8) | (gi == ng - 1 ? na_lo - gi * align : align);
      } else {
        t.pad = tail_group(j);
      }
    }
    tiles[j] = t;
  }
  // zero tiles for rows past sum(group_sizes)
  for (int z = e; z < ntail; z += blockDim.x) {  // may exceed the block when many rows are unused
    MTile t;
    t.e = -1;
    t.r0 = used + z * BM;
    t.r1 = min(used + (z + 1) * BM, M);
    t.pad = (align > 1 && merge > 0) ? tail_group(ntiles + z) : 0;
    tiles[s_total[1] + z] = t;
  }
  if (e == 0) {
    count[0] = s_total[1] + ntail;
    count[1] = s_total[1];  // tiles with an expert (the rest are zero tiles)
  }
  // expert order by descending group size (ties: lower id first), used by tgmm; count[2] = the
  // experts with rows before M is applied (a prefix of that order)
  if (need_order) {
    const int nz = __syncthreads_count(e < E && g > 0);
    if (e == 0) count[2] = nz;
  }
  if (need_order && e < E) {
    // four sizes per LDS read; entries past E hold 0 and never rank ahead (o > g fails for
    // g >= 0, and o == g needs h < e < E)
    int rank = 0;
    const int4* s4 = (const int4*)s_gs;
#pragma unroll 4
    for (int h4 = 0; h4 < (E + 3) / 4; ++h4) {
      const int4 o = s4[h4];
      const int h = 4 * h4;
      rank += (o.x > g || (o.x == g && h < e)) ? 1 : 0;
      rank += (o.y > g || (o.y == g && h + 1 < e)) ? 1 : 0;
      rank += (o.z > g || (o.z == g && h + 2 < e)) ? 1 : 0;
      rank += (o.w > g || (o.w == g && h + 3 < e)) ? 1 : 0;
    }
    order[rank] = e;
  }
}

// ---- generic exact-fp32 path ------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float gld(const T* p, int64_t i);
template <> __device__ __forceinline__ float gld<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float gld<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T> __device__ __forceinline__ void gst(T* p, int64_t i, float v);
template <> __device__ __forceinline__ void gst<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void gst<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

// MODE 0: C[r,n] = sum_k A[r,k] W[e,k,n]   (W: [E][Kred][Nout])
// MODE 1: C[r,n] = sum_k A[r,k] W[e,n,k]   (W: [E][Nout][Kred], the dlhs transpose)
// MODE 2: as MODE 0 with Nout = 2I, fused SwiGLU: the 64-column tile holds 32 gate columns
//         and the 32 matching up columns; C[r,j] = silu(gate) * up, C is [M][I].
template <typename T, int MODE>
__global__ __launch_bounds__(256) void gmm_generic_kernel(const T* __restrict__ A, const T* __restrict__ W,
                                                          const MTile* __restrict__ tiles,
                                                          const int* __restrict__ count, int64_t Kred,
                                                          int64_t Nout, T* __restrict__ C) {
  constexpr int KS = 32;  // reduction elements per step; the next step's operands load during this one
  __shared__ float As[KS][65];
  __shared__ float Bs[KS][65];
  if ((int)blockIdx.x >= count[0]) return;
  const MTile t = tiles[blockIdx.x];
  const int64_t I = Nout / 2;
  const int64_t n0 = (MODE == 2) ? (int64_t)blockIdx.y * 32 : (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  if (t.e < 0) {
    const int ncol = (MODE == 2) ? 32 : 64;
    const int64_t ldc = (MODE == 2) ? I : Nout;
    for (int i = threadIdx.x; i < 64 * ncol; i += 256) {
      const int64_t r = t.r0 + i / ncol, n = n0 + i % ncol;
      if (r < t.r1 && n < ldc) gst<T>(C, r * ldc + n, 0.0f);
    }
    return;
  }
  const T* We = W + (int64_t)t.e * Kred * Nout;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  // per thread and step: 8 elements of the 64 x KS A tile (k fastest: coalesced rows) and 8 of
  // the KS x 64 W tile (n fastest), zero outside the group / matrix
  constexpr int PT = KS * 64 / 256;
  float ra[PT], rb[PT];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int i = threadIdx.x + u * 256;
      const int kk = i % KS, rr = i / KS;
      const int64_t r = t.r0 + rr, k = k0 + kk;
      ra[u] = (r < t.r1 && k < Kred) ? gld<T>(A, r * Kred + k) : 0.0f;
      const int nn = i % 64, kb = i / 64;
      const int64_t k2 = k0 + kb;
      float b = 0.0f;
      if (MODE == 2) {
        const int64_t j = n0 + (nn & 31);
        const int64_t n = (nn < 32) ? j : I + j;
        if (j < I && k2 < Kred) b = gld<T>(We, k2 * Nout + n);
      } else {
        const int64_t n = n0 + nn;
        if (n < Nout && k2 < Kred) b = (MODE == 0) ? gld<T>(We, k2 * Nout + n) : gld<T>(We, n * Kred + k2);
      }
      rb[u] = b;
    }
  };
  load(0);
  for (int64_t k0 = 0; k0 < Kred; k0 += KS) {
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int i = threadIdx.x + u * 256;
      As[i % KS][i / KS] = ra[u];
      Bs[i / 64][i % 64] = rb[u];
    }
    __syncthreads();
    if (k0 + KS < Kred) load(k0 + KS);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  if (MODE == 2) {
    __shared__ float Cs[64][65];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) Cs[ty * 4 + i][tx * 4 + j] = acc[i][j];
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 32; i += 256) {
      const int rr = i / 32, jj = i % 32;
      const int64_t r = t.r0 + rr, j = n0 + jj;
      if (r < t.r1 && j < I) gst<T>(C, r * I + j, silu_f32(Cs[rr][jj]) * Cs[rr][32 + jj]);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = t.r0 + ty * 4 + i;
    if (r >= t.r1) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < Nout) gst<T>(C, r * Nout + n, acc[i][j]);
    }
  }
}

// dW[e,k,n] = sum_{r in group e} X[r,k] G[r,n]; grid (E, ceil(K/64), ceil(N/64))
template <typename T>
__global__ __launch_bounds__(256) void tgmm_generic_kernel(const T* __restrict__ X, const T* __restrict__ G,
                                                           const int* __restrict__ offsets, int64_t K,
                                                           int64_t N, T* __restrict__ dW) {
  __shared__ float Xs[16][65];
  __shared__ float Gs[16][65];
  const int e = blockIdx.x;
  const int64_t k0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.z * 64;
  const int64_t r0 = offsets[e], r1 = offsets[e + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int64_t rb = r0; rb < r1; rb += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int c = i % 64, rr = i / 64;
      const int64_t r = rb + rr;
      Xs[rr][c] = (r < r1 && k0 + c < K) ? gld<T>(X, r * K + k0 + c) : 0.0f;
      Gs[rr][c] = (r < r1 && n0 + c < N) ? gld<T>(G, r * N + n0 + c) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = Xs[rr][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Gs[rr][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  T* out = dW + (int64_t)e * K * N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = k0 + ty * 4 + i;
    if (k >= K) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < N) gst<T>(out, k * N + n, acc[i][j]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ h, int64_t M, int64_t I,
                                                     T* __restrict__ out) {
  const int64_t total = M * I;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / I, j = i % I;
    const float g = gld<T>(h, r * 2 * I + j), u = gld<T>(h, r * 2 * I + I + j);
    gst<T>(out, i, silu_f32(g) * u);
  }
}

// dh[r, j] = dy * up * silu'(gate), dh[r, I+j] = dy * silu(gate); silu'(g) = s (1 + g (1 - s))
template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ h, const T* __restrict__ dy,
                                                         int64_t M, int64_t I, T* __restrict__ dh) {
  const int64_t total = M * I;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / I, j = i % I;
    const float g = gld<T>(h, r * 2 * I + j), u = gld<T>(h, r * 2 * I + I + j), d = gld<T>(dy, i);
    const float s = 1.0f / (1.0f + expf(-g));
    gst<T>(dh, r * 2 * I + j, d * u * (s * (1.0f + g * (1.0f - s))));
    gst<T>(dh, r * 2 * I + I + j, d * g * s);
  }
}

// Vector forms of the two kernels above for I % 8 == 0 and 16-byte aligned rows.  The M x I/8
// chunks of eight columns are numbered row-major; a workgroup takes 512 consecutive chunks, two
// per thread 256 apart, and issues every load before its stores; loads and stores are
// non-temporal (each byte is touched once).  Q is the chunk index type: 32-bit when M * I/8 fits.
// Against one row per workgroup with plain loads (same bits), C2 / C3 / C4 shapes: swiglu 5.25 /
// 6.21 / 5.46 -> 6.13 / 6.05 / 6.27 TB/s, swiglu_bwd 5.18 / 5.94 / 5.92 -> 6.04 / 6.26 / 6.26; one
// chunk per thread or four, and persistent grids of 4-16 workgroups per CU, were slower.  Each element is computed by the same
// expression as in the scalar kernels, so the results are the same bits.
constexpr int kSwChunks = 2;  // chunks per thread
template <typename T, typename Q>
__global__ __launch_bounds__(256) void swiglu_vec_kernel(const T* __restrict__ h, int64_t M, int64_t I,
                                                         T* __restrict__ out) {
  const Q cpr = (Q)(I / 8), total = (Q)M * cpr;
  const Q step = (Q)gridDim.x * 256 * kSwChunks;
  for (Q b = (Q)blockIdx.x * 256 * kSwChunks + threadIdx.x; b < total; b += step) {
    float g[kSwChunks][8], u[kSwChunks][8];
    int64_t r[kSwChunks], c[kSwChunks];
#pragma unroll
    for (int k = 0; k < kSwChunks; ++k) {
      const Q q = min(b + (Q)(k * 256), total - 1);  // in bounds; the store below is guarded
      r[k] = (int64_t)(q / cpr);
      c[k] = 8 * (int64_t)(q - (Q)r[k] * cpr);
      ld8_nt(h + r[k] * 2 * I, c[k], g[k]);
      ld8_nt(h + r[k] * 2 * I + I, c[k], u[k]);
    }
#pragma unroll
    for (int k = 0; k < kSwChunks; ++k) {
      if (b + (Q)(k * 256) >= total) break;
      float o[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = silu_f32(g[k][q]) * u[k][q];
      st8_nt(out + r[k] * I, c[k], o);
    }
  }
}
template <typename T, typename Q>
__global__ __launch_bounds__(256) void swiglu_bwd_vec_kernel(const T* __restrict__ h, const T* __restrict__ dy,
                                                             int64_t M, int64_t I, T* __restrict__ dh) {
  const Q cpr = (Q)(I / 8), total = (Q)M * cpr;
  const Q step = (Q)gridDim.x * 256 * kSwChunks;
  for (Q b = (Q)blockIdx.x * 256 * kSwChunks + threadIdx.x; b < total; b += step) {
    float g[kSwChunks][8], u[kSwChunks][8], d[kSwChunks][8];
    int64_t r[kSwChunks], c[kSwChunks];
#pragma unroll
    for (int k = 0; k < kSwChunks; ++k) {
      const Q q = min(b + (Q)(k * 256), total - 1);
      r[k] = (int64_t)(q / cpr);
      c[k] = 8 * (int64_t)(q - (Q)r[k] * cpr);
      ld8_nt(h + r[k] * 2 * I, c[k], g[k]);
      ld8_nt(h + r[k] * 2 * I + I, c[k], u[k]);
      ld8_nt(dy + r[k] * I, c[k], d[k]);
    }
#pragma unroll
    for (int k = 0; k < kSwChunks; ++k) {
      if (b + (Q)(k * 256) >= total) break;
      float dg[8], du[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float s = 1.0f / (1.0f + expf(-g[k][q]));
        dg[q] = d[k][q] * u[k][q] * (s * (1.0f + g[k][q] * (1.0f - s)));
        du[q] = d[k][q] * g[k][q] * s;
      }
      st8_nt(dh + r[k] * 2 * I, c[k], dg);
      st8_nt(dh + r[k] * 2 * I + I, c[k], du);
    }
  }
}
// Workgroups for the vector kernels: 512 chunks each, at most 2^20 (grid-stride beyond).
static int64_t swiglu_vec_blocks(int64_t M, int64_t I) {
  return std::min<int64_t>(ceil_div(M * (I / 8), 256 * kSwChunks), int64_t(1) << 20);
}
// 32-bit chunk indices when every index the kernels form (up to total - 1 + one grid stride) fits.
static bool swiglu_vec_narrow(int64_t M, int64_t I) {
  return M * (I / 8) + swiglu_vec_blocks(M, I) * 256 * kSwChunks < (int64_t(1) << 32);
}
static bool swiglu_vec_ok(int64_t I, const void* a, const void* b, const void* c) {
  return I % 8 == 0 && I > 0 && (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0 && (uintptr_t)c % 16 == 0;
}

// ---- bf16 MFMA path -------------------------------------------------------------------------
namespace mf {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;  // native vector: SROA-friendly, unlike u32x4

constexpr int BK = 64;  // reduction elements per step; one LDS row = 128 bytes = 8 chunks

__device__ __forceinline__ int lds_off(int r, int c) { return r * 128 + ((c ^ (r & 7) ^ ((r >> 3) & 7)) << 4); }

enum { FWD = 0, DLHS = 1, TGMM = 2 };
enum { EPI_STORE = 0, EPI_SWIGLU = 1 };

__device__ __forceinline__ uint32_t u4c(const u32x4& v, int d) { return v[d]; }

// 8x8 bf16 transpose: in[i] = row i (8 consecutive columns), result j = column j (8 rows).
// Column j of rows (2i, 2i+1) sits in dword j/2 of each row, low half for even j.
template <int J>
__device__ __forceinline__ u32x4 transpose_col(const u32x4 (&in)[8]) {
  constexpr uint32_t sel = (J & 1) ? 0x07060302u : 0x05040100u;
  return u32x4{__builtin_amdgcn_perm(u4c(in[1], J / 2), u4c(in[0], J / 2), sel),
                    __builtin_amdgcn_perm(u4c(in[3], J / 2), u4c(in[2], J / 2), sel),
                    __builtin_amdgcn_perm(u4c(in[5], J / 2), u4c(in[4], J / 2), sel),
                    __builtin_amdgcn_perm(u4c(in[7], J / 2), u4c(in[6], J / 2), sel)};
}

// Transpose one 8x8 block and write its 8 columns as 16-byte chunks `kb` of LDS rows c0..c0+7.
__device__ __forceinline__ void store_transposed(char* base, const u32x4 (&in)[8], int c0, int kb) {
  *(u32x4*)(base + lds_off(c0 + 0, kb)) = transpose_col<0>(in);
  *(u32x4*)(base + lds_off(c0 + 1, kb)) = transpose_col<1>(in);
  *(u32x4*)(base + lds_off(c0 + 2, kb)) = transpose_col<2>(in);
  *(u32x4*)(base + lds_off(c0 + 3, kb)) = transpose_col<3>(in);
  *(u32x4*)(base + lds_off(c0 + 4, kb)) = transpose_col<4>(in);
  *(u32x4*)(base + lds_off(c0 + 5, kb)) = transpose_col<5>(in);
  *(u32x4*)(base + lds_off(c0 + 6, kb)) = transpose_col<6>(in);
  *(u32x4*)(base + lds_off(c0 + 7, kb)) = transpose_col<7>(in);
}

struct Args {
  const uint16_t* A;  // FWD: x [M][K]; DLHS: g [M][Kout]; TGMM: x [M][Kd]
  const uint16_t* B;  // FWD: W [E][K][N]; DLHS: W [E][N=Kin][Kout]; TGMM: g [M][N]
  uint16_t* C;
  const int* count;
  const int* offsets;
  const int* order;
  const MTile* tiles;
  int M;       // rows of A (FWD/DLHS) or of x/g (TGMM)
  int Kred;    // reduction length (FWD: Kin; DLHS: Kout); TGMM: unused
  int N;       // output columns (FWD: Kout or 2I; DLHS: Kin; TGMM: N)
  int Kd;      // TGMM: output rows per expert (K of x)
  int ldc;     // output row stride (FWD: Kout or I)
  int I;       // SwiGLU intermediate size
  int E;
  int gm;      // m-tiles per scheduling group (consecutive tiles sweep gm m-tiles, then n)
  int* split_cnt = nullptr;     // split tail (FWD/DLHS store tiles): arrival counters
  float* split_part = nullptr;  //   fp32 partials, kSplitItems slots of BM x BN per XCD
  int split_on = 0;             //   0: every tile runs whole
  int ncu_x = 32;               //   CUs per XCD (one resident 256-row workgroup per CU)
  // FWD/SWIGLU with gathered A rows: sorted row r of the group layout reads row
  // gather[r] / gather_div of A (clamped to [0, gather_rows)), i.e. the dispatch gather of
  // token rows happens in the A loads and the sorted copy is never written.
  const int32_t* gather = nullptr;
  int gather_div = 1;
  int gather_rows = 0;
  // TGMM (256-row tiles): xa > 0 gives XCD x = rem % 8 the tiles of one (nrt/xa) x (ntiles/xb)
  // rectangle of each expert's tile grid (few x and g blocks per XCD L2); 0: row-major tiles
  int xa = 0, xb = 0;
  // gmm_w4_kernel: per-XCD tile queue tickets (8 ints, zero at launch); nullptr: static ranges
  int* tickets = nullptr;
  // gmm_w4_kernel: 1 = scheduling groups of varying size, each tile's group read from the tile
  // list (MTile::pad = first m-tile << 8 | m-tiles in the group); 0 = fixed groups of gm
  int vgroup = 0;
  // gmm_w4_kernel: 1 = XCD x owns n-tiles [x*nn/8, (x+1)*nn/8) of every m-tile (nn % 8 == 0), so
  // that the eight XCDs sweep the experts together and read each A tile from HBM about once
  int nsplit = 0;
};

// ---- tile loaders ------------------------------------------------------------------------------
// Direct (reduction dim contiguous in HBM): ROWS x 64 elements, CPT 16-byte chunks per thread.
template <int ROWS, int NT>
struct DirectLoader {
  static constexpr int CPT = ROWS * 8 / NT;
  static_assert((ROWS * 8) % NT == 0, "tile split");
  u32x4 r[CPT];
  // element (row, k) at src[row_index(row) * ld + k0 + k]; rows past row_max are clamped.
  __device__ __forceinline__ void load(const uint16_t* __restrict__ src, int64_t ld, int row_base, int row_max,
                                       int k0, int tid) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int q = tid + i * NT;
      int gr = row_base + (q >> 3);
      gr = gr < row_max ? gr : row_max;
      r[i] = *(const u32x4*)(src + (int64_t)gr * ld + k0 + (q & 7) * 8);
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

// Transposed (columns contiguous in HBM): 64 reduction rows x COLS columns as 8x8 blocks.
template <int COLS, int NT>
struct TransLoader {
  static constexpr int BPT = (COLS + NT - 1) / NT;
  u32x4 r[BPT][8];
  // element (red, col) at src[(red0 + red) * ld + colmap(col)]; reductions >= red_end are 0.
  template <typename ColMap>
  __device__ __forceinline__ void load(const uint16_t* __restrict__ src, int64_t ld, int red0, int red_end,
                                       ColMap colmap, int tid) {
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int q = tid + b * NT;
      const int cb = q % (COLS / 8), kb = q / (COLS / 8);
      const bool qok = (COLS % NT == 0) || (q < COLS);
      const int gc = colmap(cb * 8);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int red = red0 + kb * 8 + i;
        r[b][i] = (qok && red < red_end) ? *(const u32x4*)(src + (int64_t)red * ld + gc) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  __device__ __forceinline__ void store(char* lds, int tid) const {
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int q = tid + b * NT;
      if ((COLS % NT != 0) && q >= COLS) continue;
      store_transposed(lds, r[b], (q % (COLS / 8)) * 8, q / (COLS / 8));
    }
  }
};

template <int BM, int BN, int WM, int WN, int MODE, int EPI>
__global__ __launch_bounds__(WM* WN * 64, 1) void gmm_mfma_kernel(Args p) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile too small");
  static_assert(EPI != EPI_SWIGLU || TN % 2 == 0, "SwiGLU pairs gate/up MFMA blocks");
  constexpr int STAGE = (BM + BN) * 128;

  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- which output tile --------------------------------------------------------------
  int e, r0, r1, col0, row0 = 0;  // FWD/DLHS: rows [r0,r1) of A; TGMM: reduction rows
  int n_tile;
  if (MODE == TGMM) {
    const int ktiles = p.Kd / BM, ntiles = p.N / BN;
    const int per_e = ktiles * ntiles;
    const int total = p.E * per_e;
    const int pid = blockIdx.x;
    const int total8 = (total + 7) & ~7;
    if (pid >= total8) return;
    const int lid = (pid & 7) * (total8 >> 3) + (pid >> 3);
    if (lid >= total) return;
    e = p.order[lid / per_e];
    const int rem = lid % per_e;
    row0 = (rem / ntiles) * BM;  // k offset within dW[e]
    n_tile = rem % ntiles;
    col0 = n_tile * BN;
    r0 = p.offsets[e];
    r1 = p.offsets[e + 1];
  } else {
    const int nn = (EPI == EPI_SWIGLU) ? (p.I / (BN / 2)) : (p.N / BN);
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
    n_tile = local / gsz;
    const MTile t = p.tiles[mt];
    e = t.e;
    r0 = t.r0;
    r1 = t.r1;
    col0 = n_tile * BN;
    if (e < 0) {  // rows past sum(group_sizes): zeros
      const int ncols = (EPI == EPI_SWIGLU) ? BN / 2 : BN;
      const int c0 = (EPI == EPI_SWIGLU) ? n_tile * (BN / 2) : col0;
      for (int i = tid; i < BM * ncols; i += NT) {
        const int r = r0 + i / ncols;
        if (r < r1) p.C[(int64_t)r * p.ldc + c0 + i % ncols] = 0;
      }
      return;
    }
  }

  // Global column of B for tile-local column c (a multiple of 8).
  const int I = p.I;
  auto b_col = [=](int c) -> int {
    if (EPI == EPI_SWIGLU) {
      const int w_ = c / WTN, within = c % WTN;
      const int half = within / (WTN / 2), off = within % (WTN / 2);
      return half * I + n_tile * (BN / 2) + w_ * (WTN / 2) + off;
    }
    return col0 + c;
  };
  auto a_col = [=](int c) -> int { return row0 + c; };

  const int nk = (MODE == TGMM) ? (r1 - r0 + BK - 1) / BK : p.Kred / BK;

  using ALoad = typename std::conditional<MODE == TGMM, TransLoader<BM, NT>, DirectLoader<BM, NT>>::type;
  using BLoad = typename std::conditional<MODE == DLHS, DirectLoader<BN, NT>, TransLoader<BN, NT>>::type;
  ALoad la;
  BLoad lb;
  const uint16_t* Bsrc = (MODE == FWD)    ? p.B + (int64_t)e * p.Kred * p.N
                         : (MODE == DLHS) ? p.B + (int64_t)e * p.N * p.Kred
                                          : p.B;

  auto issue_loads = [&](int kt) {
    if constexpr (MODE == TGMM) {
      la.load(p.A, p.Kd, r0 + kt * BK, r1, a_col, tid);
      lb.load(Bsrc, p.N, r0 + kt * BK, r1, b_col, tid);
    } else if constexpr (MODE == FWD) {
      la.load(p.A, p.Kred, r0, p.M - 1, kt * BK, tid);
      lb.load(Bsrc, p.N, kt * BK, p.Kred, b_col, tid);
    } else {
      la.load(p.A, p.Kred, r0, p.M - 1, kt * BK, tid);
      lb.load(Bsrc, p.Kred, col0, p.N - 1, kt * BK, tid);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  if (nk > 0) {
    issue_loads(0);
    la.store(lds, tid);
    lb.store(lds + BM * 128, tid);
    __syncthreads();
  }
  const int frow = lane & 31, fchunk = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const char* As = lds + (kt & 1) * STAGE;
    const char* Bs = As + BM * 128;
    const bool more = kt + 1 < nk;
    if (more) issue_loads(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *(const bf16x8*)(As + lds_off(wm * WTM + i * 32 + frow, kk * 2 + fchunk));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *(const bf16x8*)(Bs + lds_off(wn * WTN + j * 32 + frow, kk * 2 + fchunk));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      char* An = lds + ((kt + 1) & 1) * STAGE;
      la.store(An, tid);
      lb.store(An + BM * 128, tid);
    }
    __syncthreads();
  }

  // ---- epilogue: 32x32 block (i,j), lane l, acc v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32
  const int ccol = lane & 31, rhalf = (lane >> 5) * 4;
  if (MODE == TGMM) {
    uint16_t* out = p.C + (int64_t)e * p.Kd * p.N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = row0 + wm * WTM + i * 32 + 8 * (v >> 2) + rhalf + (v & 3);
          const int col = col0 + wn * WTN + j * 32 + ccol;
          out[(int64_t)row * p.N + col] = f32_to_bf16(acc[i][j][v]);
        }
  } else if (EPI == EPI_SWIGLU) {
    const int ycol0 = n_tile * (BN / 2) + wn * (WTN / 2);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN / 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = r0 + wm * WTM + i * 32 + 8 * (v >> 2) + rhalf + (v & 3);
          if (row < r1) {
            const float gt = acc[i][j][v], up = acc[i][j + TN / 2][v];
            p.C[(int64_t)row * p.ldc + ycol0 + j * 32 + ccol] = f32_to_bf16(silu_f32(gt) * up);
          }
        }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = r0 + wm * WTM + i * 32 + 8 * (v >> 2) + rhalf + (v & 3);
          if (row < r1) p.C[(int64_t)row * p.ldc + col0 + wn * WTN + j * 32 + ccol] = f32_to_bf16(acc[i][j][v]);
        }
  }
}

// Epilogue helpers of the MFMA path (bf16 outputs).
__device__ __forceinline__ uint16_t bf16_bits_hw(float f) {
  const __bf16 h = (__bf16)f;  // v_cvt_pk_bf16_f32: round-to-nearest-even
  return __builtin_bit_cast(uint16_t, h);
}
// silu(g) * u with the hardware exp2 / reciprocal (about 1e-6 relative; used for bf16 outputs).
__device__ __forceinline__ float swiglu_fast(float g, float u) {
  return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}


// ---- v3: direct-to-LDS loads, 4-stage ring, transpose reads (FWD / SWIGLU / DLHS) ----------------
// 256x256 output tile, 8 waves (2 per SIMD) with 128x64 wave tiles, BK = 32.  Every global
// load is a global_load_lds_dwordx4 straight into a 4-deep LDS ring (no staging registers, no
// ds_write, no VALU transposes); stage s is loaded three steps before it is consumed.  Layouts
// per stage (32 KB):
//   A   : 256 rows x 64 B (k-contiguous), 16-byte chunk c of row r at chunk c ^ ((r>>2)&3)
//   W   : FWD: 32 k-rows x 512 B (n-contiguous, as in HBM), chunk c of row k at c ^ 4(k&3);
//         the MFMA operand (8 consecutive k of one n per lane) is assembled with two
//         ds_read_b64_tr_b16, whose 16-lane groups return B[k0+j][n0+lane] for j = 0..3 when
//         lane r of the group addresses B[k0 + r/4][n0 + 4(r%4)].
//         DLHS: 256 n-rows x 64 B like A.
// Each lane of a load instruction writes LDS byte (M0 + 16*lane), so the swizzle is realised by
// choosing the global source of each lane.  Both swizzles make the fragment reads conflict-free.
namespace v3 {
constexpr int BKS = 32;  // reduction elements per ring stage
// Block tile BM x 256 with an NST-deep ring of stages.
template <int BM_, int NST_>
struct Cfg {
  static constexpr int BM = BM_, BN = 256, NSTAGE = NST_;
  static constexpr int PD = NSTAGE - 1;  // stages in flight ahead of the one being computed
  static constexpr int A_BYTES = BM * BKS * 2, B_BYTES = BN * BKS * 2, STAGE = A_BYTES + B_BYTES;
  static __device__ __forceinline__ int slot(int kt) {
    return (NSTAGE & (NSTAGE - 1)) == 0 ? (kt & (NSTAGE - 1)) : kt % NSTAGE;
  }
};
__device__ __forceinline__ int a_off(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }
__device__ __forceinline__ int bn_off(int k, int c) { return k * 512 + ((c ^ ((k & 3) << 2)) << 4); }
}  // namespace v3

typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;

#ifndef MTX_V3_WPE
#define MTX_V3_WPE 2
#endif
#ifndef MTX_V3_SGB
#define MTX_V3_SGB 1
#endif
template <int MODE, int EPI, int WM, int WN, int BM_, int NST_>
__global__ __launch_bounds__(WM* WN * 64, MTX_V3_WPE) void gmm_v3_kernel(Args p) {
  using v3::BKS;
  using v3::a_off;
  using v3::bn_off;
  using C = v3::Cfg<BM_, NST_>;
  constexpr int BM = C::BM, BN = C::BN, NSTAGE = C::NSTAGE, PD = C::PD;
  constexpr int A_BYTES = C::A_BYTES, B_BYTES = C::B_BYTES, STAGE = C::STAGE;
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  constexpr int A_INSTR = A_BYTES / 1024 / (NT / 64);  // load instructions per wave per stage
  constexpr int B_INSTR = B_BYTES / 1024 / (NT / 64);
  static_assert(MODE == FWD || MODE == DLHS || MODE == TGMM, "v3 mode");
  constexpr bool A_T = (MODE == TGMM);                 // A tile stored [reduction][row] (transpose reads)
  constexpr bool B_T = (MODE == FWD || MODE == TGMM);  // B tile stored [reduction][col]
  __shared__ __attribute__((aligned(1024))) char lds[NSTAGE * STAGE];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- which output tile --------------------------------------------------------------
  // FWD/DLHS: rows [r0,r1) of A, output columns from col0.  TGMM: reduction rows [r0,r1) of
  // x and g (expert e's group), output block dW[e][row0:+BM][col0:+BN]; experts are visited
  // in descending group size so that the longest reductions start first.
  int e, r0, r1, col0, n_tile, row0 = 0;
  int piece = 0, npieces = 1, split_u = 0;  // k-piece of a split tail tile (1 piece: whole tile)
  if constexpr (MODE == TGMM) {
    const int ntiles = p.N / BN, per_e = (p.Kd / BM) * ntiles;
    const int lid = blockIdx.x;
    if (lid >= p.E * per_e) return;
    e = p.order[lid / per_e];
    const int rem = lid % per_e;
    if (p.xa > 0) {  // consecutive workgroups land on consecutive XCDs: x = rem % 8 (per_e % 8 == 0)
      const int x = rem & 7, qq = rem >> 3, rh = (p.Kd / BM) / p.xa, rw = ntiles / p.xb;
      row0 = ((x % p.xa) * rh + qq / rw) * BM;
      n_tile = (x / p.xa) * rw + qq % rw;
    } else {
      row0 = (rem / ntiles) * BM;
      n_tile = rem % ntiles;
    }
    col0 = n_tile * BN;
    r0 = p.offsets[e];
    r1 = p.offsets[e + 1];
    if (r1 <= r0) {  // empty group: dW[e] = 0
      uint16_t* out = p.C + (int64_t)e * p.Kd * p.N;
      for (int i = tid; i < BM * BN / 8; i += NT) {
        const int r = i / (BN / 8), c = (i % (BN / 8)) * 8;
        *(u32x4*)(out + (int64_t)(row0 + r) * p.N + col0 + c) = u32x4{0u, 0u, 0u, 0u};
      }
      return;
    }
  } else {
    const int nn = (EPI == EPI_SWIGLU) ? (p.I / (BN / 2)) : (p.N / BN);
    const int cnt = p.count[0];
    const int total = cnt * nn;
    const int pid = blockIdx.x;
    const int total8 = (total + 7) & ~7;
    const int xcd = pid & 7, q = pid >> 3, per = total8 >> 3;
    int lid;
    if (EPI == EPI_STORE && BM == 256 && MODE != TGMM && p.split_on) {
      // XCD xcd runs tiles [xcd*per, xcd*per + tx) in dispatch order q; when its last round is
      // at most half full (rem tiles on ncu_x CUs), those rem tiles are split along K into S
      // pieces, dispatched after the whole tiles
      const int tx = max(0, min(per, total - xcd * per));
      const int rem = tx % p.ncu_x;
      int S = (rem > 0 && rem <= kSplitMaxRem && 2 * rem <= p.ncu_x) ? min(kSplitMaxS, p.ncu_x / rem) : 1;
      S = min(S, max(p.Kred / BKS, 1));
      const int nwhole = (S > 1) ? tx - rem : tx;
      if (q >= nwhole + (S > 1 ? rem * S : 0)) return;
      if (q < nwhole) {
        lid = xcd * per + q;
      } else {
        split_u = (q - nwhole) / S;
        piece = (q - nwhole) % S;
        npieces = S;
        lid = xcd * per + nwhole + split_u;
      }
    } else {
      if (pid >= total8) return;
      lid = xcd * per + q;
      if (lid >= total) return;
    }
    const int GM = p.gm;
    const int grp = lid / (GM * nn);
    const int first_m = grp * GM;
    const int gsz = min(GM, cnt - first_m);
    const int local = lid - grp * GM * nn;
    const int mt = first_m + local % gsz;
    n_tile = local / gsz;
    const MTile t = p.tiles[mt];
    e = t.e;
    r0 = t.r0;
    r1 = t.r1;
    col0 = n_tile * BN;
    if (e < 0) {
      if (piece > 0) return;
      const int ncols = (EPI == EPI_SWIGLU) ? BN / 2 : BN;
      const int c0 = (EPI == EPI_SWIGLU) ? n_tile * (BN / 2) : col0;
      for (int i = tid; i < BM * ncols; i += NT) {
        const int r = r0 + i / ncols;
        if (r < r1) p.C[(int64_t)r * p.ldc + c0 + i % ncols] = 0;
      }
      return;
    }
  }

  // k-stages [kb0, kb0 + nk) of this workgroup (piece of npieces; the whole range when 1)
  const int nk_all = (MODE == TGMM) ? (r1 - r0 + BKS - 1) / BKS : p.Kred / BKS;
  const int kb0 = piece * nk_all / npieces;
  const int nk = (piece + 1) * nk_all / npieces - kb0;
  const int tail = (MODE == TGMM) ? (r1 - r0) - (nk - 1) * BKS : BKS;  // rows in the last step

  // ---- per-lane global sources of the load instructions (byte offsets at k-step 0) -----
  // A row-major operand (FWD/DLHS): lane l of segment s fills row 16s + l/4, chunk slot l%4.
  // Transposed operands (W in FWD, x and g in TGMM): lane l fills reduction row 2s + l/32,
  // chunk slot l%32.  TGMM rows are expert-relative and clamped to M-1 at issue time (the
  // reduction tail past r1 is zeroed in the fragments).
  const char* Ab = (const char*)p.A;
  const char* Bb = (MODE == TGMM) ? (const char*)p.B : (const char*)(p.B + (int64_t)e * p.Kred * p.N);
  uint32_t aoff[A_INSTR], boff[B_INSTR];
  int arow[A_T ? A_INSTR : 1], brow[(MODE == TGMM) ? B_INSTR : 1];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int seg = wave * A_INSTR + i;  // 1 KB segment of the A region
    if constexpr (A_T) {
      const int k = seg * 2 + (lane >> 5), pc = lane & 31;
      const int c = pc ^ ((k & 3) << 2);
      arow[i] = r0 + k;
      aoff[i] = (uint32_t)(row0 + c * 8) * 2u;
    } else {
      const int r = seg * 16 + (lane >> 2), pc = lane & 3;
      const int c = pc ^ ((r >> 2) & 3);
      // rows past the tile's group repeat its last row: never used, and cache hits
      int gr = r0 + r;
      gr = gr < r1 ? gr : r1 - 1;
      if (MODE == FWD && p.gather) gr = min(max(p.gather[gr], 0) / p.gather_div, p.gather_rows - 1);
      aoff[i] = ((uint32_t)gr * (uint32_t)p.Kred + (uint32_t)(c * 8)) * 2u;
    }
  }
#pragma unroll
  for (int i = 0; i < B_INSTR; ++i) {
    const int seg = wave * B_INSTR + i;
    if constexpr (B_T) {
      const int k = seg * 2 + (lane >> 5), pc = lane & 31;
      const int c = pc ^ ((k & 3) << 2);
      const int tc = c * 8;  // tile-local column
      int gc;
      if (EPI == EPI_SWIGLU) {
        const int w_ = tc / WTN, within = tc % WTN;
        const int half = within / (WTN / 2), o = within % (WTN / 2);
        gc = half * p.I + n_tile * (BN / 2) + w_ * (WTN / 2) + o;
      } else {
        gc = col0 + tc;
      }
      if constexpr (MODE == TGMM) {
        brow[i] = r0 + k;
        boff[i] = (uint32_t)gc * 2u;
      } else {
        boff[i] = ((uint32_t)k * (uint32_t)p.N + (uint32_t)gc) * 2u;
      }
    } else {
      const int r = seg * 16 + (lane >> 2), pc = lane & 3;
      const int c = pc ^ ((r >> 2) & 3);
      boff[i] = ((uint32_t)(col0 + r) * (uint32_t)p.Kred + (uint32_t)(c * 8)) * 2u;
    }
  }
  const uint32_t a_step = BKS * 2;
  const uint32_t b_step = B_T ? (uint32_t)BKS * (uint32_t)p.N * 2u : (uint32_t)BKS * 2u;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char*)lds;
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const int mlast = p.M - 1;
  // Stages past the end re-read the last one (in bounds) into a ring slot that is no longer
  // read, which keeps the main loop free of branches.
  auto issue_stage = [&](int kt_) {
    const uint32_t st = lds_base + (uint32_t)(C::slot(kt_) * STAGE);
    const int kt = kb0 + min(kt_, nk - 1);
    if constexpr (MODE == TGMM) {
#pragma unroll
      for (int i = 0; i < A_INSTR; ++i) {
        const uint32_t row = (uint32_t)min(arow[i] + kt * BKS, mlast);
        gload_lds16(Ab + row * (uint32_t)(p.Kd * 2) + aoff[i], st + (wave_u * A_INSTR + i) * 1024u);
      }
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i) {
        const uint32_t row = (uint32_t)min(brow[i] + kt * BKS, mlast);
        gload_lds16(Bb + row * (uint32_t)(p.N * 2) + boff[i], st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_INSTR; ++i)
        gload_lds16(Ab + aoff[i] + (uint32_t)kt * a_step, st + (wave_u * A_INSTR + i) * 1024u);
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i)
        gload_lds16(Bb + boff[i] + (uint32_t)kt * b_step, st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
    }
  };

  // ---- fragments ---------------------------------------------------------------------
  bf16x8 fa[2][TM], fb[2][TN];
  const int frow = lane & 31, fhalf = lane >> 5;
  // One 32-wide MFMA operand from a [reduction][col] tile via two transpose reads: lane l gets
  // reduction rows kk*16 + 8*(l/32) + 0..7 of column c0 + l%32.
  auto read_tr = [&](const char* region, int c0, int kk) -> bf16x8 {
    const int n = c0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int k = kk * 16 + 8 * fhalf + ((lane & 15) >> 2);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k, n >> 3) + (n & 7) * 2));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k + 4, n >> 3) + (n & 7) * 2));
    const s16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
  };
  auto read_frags = [&](int kt, int kk, int buf, int nb) {
    // a wave with no rows of the group in this tile (small groups) runs no MFMA: no reads
    if (MODE != TGMM && nb == 0) return;
    const char* st = lds + C::slot(kt) * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if (i >= nb) continue;
      if constexpr (A_T) {
        fa[buf][i] = read_tr(st, wm * WTM + i * 32, kk);
      } else {
        const int r = wm * WTM + i * 32 + frow;
        fa[buf][i] = *(const bf16x8*)(st + a_off(r, kk * 2 + fhalf));
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (B_T) {
        fb[buf][j] = read_tr(st + A_BYTES, wn * WTN + j * 32, kk);
      } else {
        const int r = wn * WTN + j * 32 + frow;
        fb[buf][j] = *(const bf16x8*)(st + A_BYTES + a_off(r, kk * 2 + fhalf));
      }
    }
  };
  // TGMM reduction tail: keep only the first `rem` rows of the last step (both operands, so
  // rows of other groups never reach the accumulators).
  auto mask_frags = [&](int buf, int kk, int rem) {
    const int nv = min(max(rem - kk * 16 - 8 * fhalf, 0), 8);
    u32x4 m;
#pragma unroll
    for (int d = 0; d < 4; ++d) m[d] = (2 * d + 1 < nv) ? 0xFFFFFFFFu : ((2 * d < nv) ? 0xFFFFu : 0u);
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[buf][i] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, fa[buf][i]) & m);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[buf][j] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, fb[buf][j]) & m);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  constexpr int LPS = A_INSTR + B_INSTR;  // load instructions per stage per thread
  // prologue: stages 0..PD-1 in flight; stages 0 and 1 landed and visible
#pragma unroll
  for (int s = 0; s < PD; ++s) issue_stage(s);
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));  // (vmcnt counts outstanding loads)
  __syncthreads();
  // 32-row blocks of this wave that hold rows of the group (FWD/DLHS tiles of small groups
  // are partly empty): MFMAs and A reads of empty blocks are skipped.
  const int nbi = (MODE == TGMM) ? TM : min(max((r1 - r0 - wm * WTM + 31) / 32, 0), TM);
  read_frags(0, 0, 0, nbi);

  auto main_loop = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    const int nb = FULL ? TM : nbi;
    for (int kt = 0; kt < nk; ++kt) {
      issue_stage(kt + PD);
#if MTX_V3_SGB
      if constexpr (FULL && MODE != TGMM) {
        // explicit interleave: one fragment read of the next substep after each MFMA
        __builtin_amdgcn_sched_barrier(0);
        read_frags(kt, 1, 1, nb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int q = 0; q < TM * TN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        read_frags(kt + 1, 0, 0, nb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int q = 0; q < TM * TN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
        __builtin_amdgcn_s_barrier();  // no LDS-read wait: see below
        continue;
      }
#endif
      // substep 0: prefetch substep 1 of this stage
      read_frags(kt, 1, 1, nb);
      if (MODE == TGMM && tail < BKS && kt == nk - 1) mask_frags(0, 0, tail);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (!FULL && i >= nb) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
      }
      // substep 1: prefetch substep 0 of the next stage (visible since the last barrier).  On
      // the last step this reads an unused ring slot: in bounds, and branch-free so that the
      // MFMAs below only wait for the fragments they use.
      read_frags(kt + 1, 0, 0, nb);
      if (MODE == TGMM && tail < BKS && kt == nk - 1) mask_frags(1, 1, tail);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (!FULL && i >= nb) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
      }
      // stage kt+2 must have landed before the barrier makes it visible to every wave (later
      // stages, possibly re-reads past the end, may still be in flight).  A bare s_barrier:
      // __syncthreads() would also wait for this wave's outstanding LDS reads, which are
      // fragments of stage kt+1 (visible since the previous barrier); the slot refilled next
      // (stage kt's, by iteration kt+1) was read only by fragments this iteration's MFMAs used.
      __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
      __builtin_amdgcn_s_barrier();
    }
  };
  // Both loop versions execute the same barriers, so waves of one workgroup may take either.
  if (MODE == TGMM || nbi == TM) main_loop(std::integral_constant<bool, true>());
  else main_loop(std::integral_constant<bool, false>());
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));  // no ring load may land after the workgroup ends

  if (npieces > 1) {
    // Split tail piece: publish the fp32 partial tile; the piece that arrives last (by the
    // tile's counter) reloads every piece and adds them in piece order -- the same sum
    // whatever the arrival order -- then runs the epilogue.  Nothing waits on another
    // workgroup.  A lane's partial is float4 chunks, one coalesced 1 KB row per wave store.
    static_assert(BM * BN <= kSplitSlotFloats, "split slot");
    typedef __attribute__((ext_vector_type(4))) float f32x4;
    constexpr int64_t SLOT4 = kSplitSlotFloats / 4;
    const int xcd_e = (int)(blockIdx.x & 7);
    f32x4* part = (f32x4*)(p.split_part + (int64_t)(xcd_e * kSplitItems + split_u * npieces) * kSplitSlotFloats);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          part[piece * SLOT4 + ((i * TN + j) * 4 + g) * NT + tid] =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(p.split_cnt + xcd_e * kSplitMaxRem + split_u, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == npieces - 1;
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#pragma unroll
    for (int s2 = 0; s2 < kSplitMaxS; ++s2) {  // unrolled: each piece's loads issue together
      if (s2 >= npieces) break;
      const f32x4* src = part + s2 * SLOT4;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 v = src[((i * TN + j) * 4 + g) * NT + tid];
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[i][j][4 * g + c] = (s2 == 0) ? v[c] : acc[i][j][4 * g + c] + v[c];
          }
    }
  }

  // ---- epilogue: the MFMAs computed C^T blocks (operands swapped), so acc[i][j][4g+q] of lane
  // l is C[row i*32 + l%32][col j*32 + 8g + 4(l/32) + q]: four consecutive columns per lane.
  // The tile is staged in the (now idle) ring as packed bf16 rows, 16-byte chunk c of row r at
  // chunk c ^ (r & 15), and written back with 16 contiguous bytes per lane so that every row
  // of the tile goes out as whole 128-byte lines.
  constexpr int OCOLS = (EPI == EPI_SWIGLU) ? BN / 2 : BN;  // bf16 output columns of the tile
  constexpr int OROW = OCOLS * 2;                           // staged row bytes
  constexpr int OCH = OROW / 16;                            // 16-byte chunks per row
  static_assert(BM * OROW <= NSTAGE * STAGE, "staging fits the ring");
  auto pack4 = [](float a, float b, float c, float d) -> bf16x4 {
    return bf16x4{(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
  };
  auto stage8 = [&](int r, int col, bf16x4 v) {  // col: tile column, multiple of 4
    const int c = col >> 3;
    *(bf16x4*)(lds + r * OROW + ((c ^ (r & 15)) << 4) + (col & 7) * 2) = v;
  };
  __syncthreads();  // every wave is done with the ring
  {
    const int frow = lane & 31, h4 = 4 * (lane >> 5);
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN / 2; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x16& gt = acc[i][j];
            const f32x16& up = acc[i][j + TN / 2];
            stage8(wm * WTM + i * 32 + frow, wn * (WTN / 2) + j * 32 + 8 * g + h4,
                   pack4(swiglu_fast(gt[4 * g], up[4 * g]), swiglu_fast(gt[4 * g + 1], up[4 * g + 1]),
                         swiglu_fast(gt[4 * g + 2], up[4 * g + 2]), swiglu_fast(gt[4 * g + 3], up[4 * g + 3])));
          }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            stage8(wm * WTM + i * 32 + frow, wn * WTN + j * 32 + 8 * g + h4,
                   pack4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]));
    }
  }
  __syncthreads();
  uint16_t* obase;
  int64_t ld;
  int rbase, rlimit;
  if constexpr (MODE == TGMM) {
    obase = p.C + (int64_t)e * p.Kd * p.N + col0;
    ld = p.N;
    rbase = row0;
    rlimit = row0 + BM;
  } else {
    obase = p.C + ((EPI == EPI_SWIGLU) ? n_tile * (BN / 2) : col0);
    ld = p.ldc;
    rbase = r0;
    rlimit = r1;
  }
  constexpr int RPI = 64 / OCH;  // rows per wave instruction
  for (int rr = wave * RPI + lane / OCH; rr < BM; rr += NT / OCH) {
    const int c = lane % OCH;
    const u32x4 v = *(const u32x4*)(lds + rr * OROW + ((c ^ (rr & 15)) << 4));
    const int row = rbase + rr;
    if (row < rlimit) *(u32x4*)(obase + (int64_t)row * ld + c * 8) = v;
  }
}

// ---- v4p: persistent workgroups whose ring runs across tiles (FWD / DLHS, plain store) --------
// With short reductions (a few dozen 32-k stages per tile) the ring fill at every tile start and
// the dispatch gap between workgroups cost 10-15 % of a 256x256 tile.  This kernel computes the
// same tiles with the same waves, ring, fragments and MFMA order as gmm_v3_kernel (the same bits),
// but each workgroup (at most one per CU) walks its XCD's tile range and keeps issuing ring loads
// across tile boundaries, so the next tile's first three stages are in flight while the current
// tile's epilogue stores.  The tile list is read through the scalar cache, so that a tile switch
// waits on lgkmcnt, never on the ring's vmcnt; the epilogue stages each wave's 32 x 64 blocks in
// its own 4 KB of the tile's last (consumed) ring slot.  Needs Kred >= 4 stages.
template <int MODE>
__global__ __launch_bounds__(512, 2) void gmm_v4p_kernel(Args p) {
  using v3::BKS;
  using v3::a_off;
  using v3::bn_off;
  using Cf = v3::Cfg<256, 4>;
  constexpr int BN = Cf::BN, NSTAGE = Cf::NSTAGE, PD = Cf::PD;
  constexpr int A_BYTES = Cf::A_BYTES, STAGE = Cf::STAGE;
  constexpr int WN = 4, WTM = 128, WTN = 64, TM = 4, TN = 2;
  constexpr int A_INSTR = 2, B_INSTR = 2, LPS = A_INSTR + B_INSTR;
  static_assert(MODE == FWD || MODE == DLHS, "v4p mode");
  static_assert(Cf::BM == 256 && A_BYTES == 16384 && Cf::B_BYTES == 16384 && NSTAGE == 4, "v4p ring");
  constexpr bool B_T = (MODE == FWD);  // B tile stored [reduction][col]
  __shared__ __attribute__((aligned(1024))) char lds[NSTAGE * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const int wm = wave / WN, wn = wave % WN;
  const int nn = p.N / BN;
  const int cnt = p.count[0];
  const int total = cnt * nn;
  // XCD x (= blockIdx % 8) walks tiles [x*per, (x+1)*per) with its gridDim/8 workgroups
  const int nx = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), q = (int)(blockIdx.x >> 3);
  const int per = (total + 7) >> 3;
  const int lid_end = min((xcd + 1) * per, total);
  int lid = xcd * per + q;
  if (lid >= lid_end) return;
  const int nk = p.Kred / BKS;

  struct Tile {
    int e, r0, r1, n_tile, zero;
  };
  auto decode = [&](int l) -> Tile {
    const int GM = p.gm;
    const int grp = l / (GM * nn);
    const int first_m = grp * GM;
    const int gsz = min(GM, cnt - first_m);
    const int local = l - grp * GM * nn;
    // read-only tile list through the scalar cache (constant address space, uniform index)
    typedef const __attribute__((address_space(4))) int cint_t;
    const int mt = __builtin_amdgcn_readfirstlane(first_m + local % gsz);
    const cint_t* tp = (const cint_t*)(uintptr_t)(p.tiles + mt);
    Tile T;
    const int e = tp[0];
    T.zero = e < 0;
    T.e = e < 0 ? 0 : e;  // rows past sum(group_sizes): computed with expert 0, stored as 0
    T.r0 = tp[1];
    T.r1 = tp[2];
    T.n_tile = local / gsz;
    return T;
  };
  // per-lane 32-bit byte offsets of the load instructions at k-stage 0 (the v3 layout), and the
  // tile's uniform weight base
  struct Src {
    uint32_t aoff[A_INSTR], boff[B_INSTR];
    const char* B;
  };
  auto make_src = [&](const Tile& T) -> Src {
    Src S;
    const int col0 = T.n_tile * BN;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      const int seg = wave * A_INSTR + i;
      const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
      const int gr = min(T.r0 + r, T.r1 - 1);  // rows past the group repeat its last row
      S.aoff[i] = ((uint32_t)gr * (uint32_t)p.Kred + (uint32_t)(c * 8)) * 2u;
    }
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
      const int seg = wave * B_INSTR + i;
      if constexpr (B_T) {
        const int k = seg * 2 + (lane >> 5), c = (lane & 31) ^ ((k & 3) << 2);
        S.boff[i] = ((uint32_t)k * (uint32_t)p.N + (uint32_t)(col0 + c * 8)) * 2u;
      } else {
        const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
        S.boff[i] = ((uint32_t)(col0 + r) * (uint32_t)p.Kred + (uint32_t)(c * 8)) * 2u;
      }
    }
    S.B = (const char*)(p.B + (int64_t)T.e * p.Kred * p.N);
    return S;
  };

  Tile cur = decode(lid);
  int lid_next = lid + nx;
  Tile nxt = lid_next < lid_end ? decode(lid_next) : cur;
  // sources of the tile whose stages are being issued: the current tile's until its last stage
  // is issued, then the next tile's (the last tile's steps past its end re-read its first
  // stages: in bounds, into slots that are never read)
  Src src = make_src(cur);

  const uint32_t lds_base = lds_addr(lds);
  const int64_t b_step = B_T ? (int64_t)BKS * p.N * 2 : (int64_t)BKS * 2;
  // ring step g: stage k of the tile whose sources are in src
  auto issue = [&](int g, int k) {
    const uint32_t st = lds_base + (uint32_t)((g & (NSTAGE - 1)) * STAGE);
    const char* A = (const char*)p.A + (int64_t)k * (BKS * 2);
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) gload_lds16_s(A, src.aoff[i], st + (wave_u * A_INSTR + i) * 1024u);
    const char* B = src.B + (int64_t)k * b_step;
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i)
      gload_lds16_s(B, src.boff[i], st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
  };

  // ---- fragments (the v3 reads, by ring step) ---------------------------------------------
  bf16x8 fa[2][TM], fb[2][TN];
  const int frow = lane & 31, fhalf = lane >> 5;
  auto read_tr = [&](const char* region, int c0, int kk) -> bf16x8 {
    const int n = c0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int k = kk * 16 + 8 * fhalf + ((lane & 15) >> 2);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k, n >> 3) + (n & 7) * 2));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k + 4, n >> 3) + (n & 7) * 2));
    const s16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
  };
  auto read_frags = [&](int g_, int kk, int buf, int nb) {
    if (nb == 0) return;  // a wave with no rows of the group in this tile runs no MFMA
    const char* st = lds + (g_ & (NSTAGE - 1)) * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if (i >= nb) continue;
      const int r = wm * WTM + i * 32 + frow;
      fa[buf][i] = *(const bf16x8*)(st + a_off(r, kk * 2 + fhalf));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (B_T) {
        fb[buf][j] = read_tr(st + A_BYTES, wn * WTN + j * 32, kk);
      } else {
        const int r = wn * WTN + j * 32 + frow;
        fb[buf][j] = *(const bf16x8*)(st + A_BYTES + a_off(r, kk * 2 + fhalf));
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // prologue: ring steps 0..PD-1 in flight; steps 0 and 1 landed and visible
#pragma unroll
  for (int s = 0; s < PD; ++s) issue(s, s);
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
  __syncthreads();
  int g = 0;

  for (;;) {
    // 32-row blocks of this wave that hold rows of the tile (wave-uniform, so that the ring step
    // g updated under the branch below stays in a scalar register)
    const int nbi = __builtin_amdgcn_readfirstlane(min(max((cur.r1 - cur.r0 - wm * WTM + 31) / 32, 0), TM));
    read_frags(g, 0, 0, nbi);
    auto tile_loop = [&](auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
      const int nb = FULL ? TM : nbi;
      for (int kt = 0; kt < nk; ++kt, ++g) {
        if (kt + PD == nk) src = make_src(nxt);  // from here on the ring loads the next tile
        issue(g + PD, kt + PD < nk ? kt + PD : kt + PD - nk);
        if constexpr (FULL) {
          // explicit interleave: one fragment read of the next substep after each MFMA
          __builtin_amdgcn_sched_barrier(0);
          read_frags(g, 1, 1, nb);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
#pragma unroll
          for (int qq = 0; qq < TM * TN; ++qq) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
          read_frags(g + 1, 0, 0, nb);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
#pragma unroll
          for (int qq = 0; qq < TM * TN; ++qq) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
        } else {
          read_frags(g, 1, 1, nb);
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            if (i >= nb) continue;
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[0][j], fa[0][i], acc[i][j], 0, 0, 0);
          }
          read_frags(g + 1, 0, 0, nb);
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            if (i >= nb) continue;
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
          }
        }
        // step g+2 landed (g+3 may be in flight); bare barrier as in v3: the slot refilled next
        // was read only by fragments that this step's MFMAs consumed
        __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
        __builtin_amdgcn_s_barrier();
      }
    };
    // both loop versions execute the same barriers, so the waves of a workgroup may take either
    if (nbi == TM) tile_loop(std::integral_constant<bool, true>());
    else tile_loop(std::integral_constant<bool, false>());

    // ---- epilogue: the tile's last ring slot (step g-1) is consumed and is refilled only by the
    // next tile's first ring load; every wave's fragment reads of it must complete before the
    // staging writes (the bare barriers do not order them): LDS-only release fence, barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    // acc[i][j][4q+c] of lane l is C[row i*32 + l%32][col j*32 + 8q + 4(l/32) + c]; each wave
    // stages 32 rows x 64 columns (4 KB, 16-byte chunk c of row r at chunk c ^ (r & 7)) and writes
    // them back as whole 128-byte rows
    char* wst = lds + ((g - 1) & (NSTAGE - 1)) * STAGE + wave * 4096;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const bf16x4 v = cur.zero ? bf16x4{(__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f}
                                    : bf16x4{(__bf16)acc[i][j][4 * gq], (__bf16)acc[i][j][4 * gq + 1],
                                             (__bf16)acc[i][j][4 * gq + 2], (__bf16)acc[i][j][4 * gq + 3]};
          *(bf16x4*)(wst + frow * 128 + (((4 * j + gq) ^ (frow & 7)) << 4) + 8 * fhalf) = v;
        }
      __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int rloc = rr * 8 + (lane >> 3);
        const u32x4 v = *(const u32x4*)(wst + rloc * 128 + (((lane & 7) ^ (rloc & 7)) << 4));
        const int row = cur.r0 + wm * WTM + i * 32 + rloc;
        if (row < cur.r1) *(u32x4*)(p.C + (int64_t)row * p.ldc + cur.n_tile * BN + wn * WTN + (lane & 7) * 8) = v;
      }
      __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);  // reads done before the next block overwrites
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    // the staging slot is the next tile's first ring load target: every wave's reads of it done
    // (LDS-only, so the ring's loads in flight are not waited for)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();

    // ---- next tile ------------------------------------------------------------------------
    lid = lid_next;
    if (lid >= lid_end) break;
    cur = nxt;
    lid_next = lid + nx;
    if (lid_next < lid_end) nxt = decode(lid_next);
  }
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));  // the last steps' re-read loads land before exit
}

// ---- tgmm_v4p: persistent tgmm (256x256 tiles) ----------------------------------------------------
// The tiles, waves, ring, transposed DMA layouts, fragment reads, reduction-tail masking and MFMA
// order of gmm_v3_kernel in TGMM mode (the same bits), with one workgroup per CU and the ring
// running across tiles: the next tile's first three stages are loaded during the current tile's
// last three, so a tile starts without the ring prologue.  Tiles come in the v3 order (experts by
// descending group size, XCD x = tile % 8 with the xa x xb XCD rectangles); the count[2] experts
// with rows (a prefix of that order) are computed here, XCD x's workgroups taking their first
// tile statically and the rest from the XCD's ticket counter count[4 + x], drawn by wave 0 at the
// start of each epilogue: the first epilogue draws two (the next tile and the one after), every
// later one one, so that a workgroup holds at most one tile beyond the current one.  The ring
// runs on into the next tile when both have three or more stages (the three-stage lookahead then
// stays within it); otherwise the lookahead re-reads the current tile's last stage into slots that
// are not read and the ring restarts.  The zero tiles of the other experts are written first.  A
// tile's loads need no per-lane state beyond its uniform (r0, row0, col0): lane l of segment s
// loads reduction row 2s + l/32 (clamped to M-1) at chunk slot l%32.
__global__ __launch_bounds__(512, 2) void tgmm_v4p_kernel(Args p) {
  using v3::BKS;
  using v3::bn_off;
  using Cf = v3::Cfg<256, 4>;
  constexpr int BM = Cf::BM, BN = Cf::BN, NSTAGE = Cf::NSTAGE, PD = Cf::PD;
  constexpr int A_BYTES = Cf::A_BYTES, STAGE = Cf::STAGE;
  constexpr int WN = 4, WTM = 128, WTN = 64, TM = 4, TN = 2;
  constexpr int A_INSTR = 2, B_INSTR = 2, LPS = A_INSTR + B_INSTR;
  static_assert(A_BYTES == 16384 && Cf::B_BYTES == 16384 && NSTAGE == 4 && PD == 3, "tgmm_v4p ring");
  __shared__ __attribute__((aligned(1024))) char lds[NSTAGE * STAGE];
  __shared__ int s_ticket;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const int wm = wave / WN, wn = wave % WN;
  const int nr = p.Kd / BM, nc = p.N / BN, per_e = nr * nc;
  typedef const __attribute__((address_space(4))) int cint_t;
  const int n_rows = __builtin_amdgcn_readfirstlane(((const cint_t*)(uintptr_t)p.count)[2]);
  const int total = n_rows * per_e, all = p.E * per_e;
  const int nx = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), q = (int)(blockIdx.x >> 3);

  struct Tile {
    int e, row0, col0, r0, nk, tail;
  };
  // tile lid of the v3 order; the read-only lists go through the scalar cache.  An expert whose
  // rows were all dropped (past M) still has one stage, wholly masked: its tile stores zeros.
  auto decode = [&](int lid) -> Tile {
    Tile T;
    const int ei = lid / per_e, rem = lid - ei * per_e;
    T.e = __builtin_amdgcn_readfirstlane(((const cint_t*)(uintptr_t)p.order)[ei]);
    int n_tile;
    if (p.xa > 0) {
      const int x = rem & 7, qq = rem >> 3, rh = nr / p.xa, rw = nc / p.xb;
      T.row0 = ((x % p.xa) * rh + qq / rw) * BM;
      n_tile = (x / p.xa) * rw + qq % rw;
    } else {
      T.row0 = (rem / nc) * BM;
      n_tile = rem % nc;
    }
    T.col0 = n_tile * BN;
    const cint_t* ofs = (const cint_t*)(uintptr_t)p.offsets;
    T.r0 = __builtin_amdgcn_readfirstlane(ofs[T.e]);
    const int rows = max(__builtin_amdgcn_readfirstlane(ofs[T.e + 1]) - T.r0, 0);
    T.nk = max((rows + BKS - 1) / BKS, 1);
    T.tail = rows - (T.nk - 1) * BKS;
    return T;
  };

  // ---- the zero tiles of the experts without rows (no LDS) ---------------------------------------
  for (int lid = total + (int)blockIdx.x; lid < all; lid += (int)gridDim.x) {
    const Tile T = decode(lid);
    uint16_t* out = p.C + (int64_t)T.e * p.Kd * p.N + (int64_t)T.row0 * p.N + T.col0;
    for (int i = tid; i < BM * BN / 8; i += 512) {
      const int r = i / (BN / 8), c = (i % (BN / 8)) * 8;
      *(u32x4*)(out + (int64_t)r * p.N + c) = u32x4{0u, 0u, 0u, 0u};
    }
  }

  // per-lane load constants: reduction row kl[i] of segment wave*2+i, column offset cb[i] (bytes)
  int kl[2];
  uint32_t cb[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    kl[i] = (wave * 2 + i) * 2 + (lane >> 5);
    cb[i] = (uint32_t)(((lane & 31) ^ ((kl[i] & 3) << 2)) * 16);
  }
  const uint32_t lds_base = lds_addr(lds);
  const int mlast = p.M - 1;
  const uint32_t lda = (uint32_t)p.Kd * 2u, ldb = (uint32_t)p.N * 2u;
  Tile cur{}, nxt{}, la{};  // la: the tile the lookahead loads (nxt when the ring runs on, else cur)
  // ring step g: stage kt counted from the current tile's start (past its end: the lookahead tile's
  // stage, clamped to its last)
  auto issue = [&](int g, int kt) {
    const bool in = kt < cur.nk;
    const int k = in ? kt : min(kt - cur.nk, la.nk - 1);
    const int r0 = in ? cur.r0 : la.r0, row0 = in ? cur.row0 : la.row0, col0 = in ? cur.col0 : la.col0;
    const uint32_t st = lds_base + (uint32_t)((g & (NSTAGE - 1)) * STAGE);
    const int rb = r0 + k * BKS;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      const uint32_t row = (uint32_t)min(rb + kl[i], mlast);
      gload_lds16_s(p.A, row * lda + (uint32_t)row0 * 2u + cb[i], st + (wave_u * A_INSTR + i) * 1024u);
    }
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
      const uint32_t row = (uint32_t)min(rb + kl[i], mlast);
      gload_lds16_s(p.B, row * ldb + (uint32_t)col0 * 2u + cb[i], st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
    }
  };

  // ---- fragments (the v3 TGMM reads, by ring step) ------------------------------------------------
  bf16x8 fa[2][TM], fb[2][TN];
  const int frow = lane & 31, fhalf = lane >> 5;
  auto read_tr = [&](const char* region, int c0, int kk) -> bf16x8 {
    const int n = c0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int k = kk * 16 + 8 * fhalf + ((lane & 15) >> 2);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k, n >> 3) + (n & 7) * 2));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k + 4, n >> 3) + (n & 7) * 2));
    const s16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
  };
  auto read_frags = [&](int g_, int kk, int buf) {
    const char* st = lds + (g_ & (NSTAGE - 1)) * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[buf][i] = read_tr(st, wm * WTM + i * 32, kk);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[buf][j] = read_tr(st + A_BYTES, wn * WTN + j * 32, kk);
  };
  // reduction tail: keep only the first `rem` rows of the tile's last stage (both operands)
  auto mask_frags = [&](int buf, int kk, int rem) {
    const int nv = min(max(rem - kk * 16 - 8 * fhalf, 0), 8);
    u32x4 m;
#pragma unroll
    for (int d = 0; d < 4; ++d) m[d] = (2 * d + 1 < nv) ? 0xFFFFFFFFu : ((2 * d < nv) ? 0xFFFFu : 0u);
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[buf][i] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, fa[buf][i]) & m);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[buf][j] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, fb[buf][j]) & m);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  int g = 0;
  // ring prologue at the current tile: steps 0..PD-1 in flight, 0 and 1 landed and visible
  auto prologue = [&]() {
    g = 0;
#pragma unroll
    for (int s2 = 0; s2 < PD; ++s2) issue(s2, s2);
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
    __syncthreads();
    read_frags(0, 0, 0);
  };

  auto valid = [&](int jj) { return 8 * jj + xcd < total; };
  int j = q;
  if (valid(j)) {
    int j_next = -1;
    cur = decode(8 * j + xcd);
    la = cur;
    bool chain = false;
    prologue();
    for (;;) {
      const int nk = cur.nk, tail = cur.tail;
      for (int kt = 0; kt < nk; ++kt, ++g) {
        issue(g + PD, kt + PD);
        read_frags(g, 1, 1);
        if (tail < BKS && kt == nk - 1) mask_frags(0, 0, tail);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < TN; ++jj)
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[0][jj], fa[0][i], acc[i][jj], 0, 0, 0);
        // the next step's first fragments: the next stage of this tile, or of the next one
        read_frags(g + 1, 0, 0);
        if (tail < BKS && kt == nk - 1) mask_frags(1, 1, tail);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < TN; ++jj)
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[1][jj], fa[1][i], acc[i][jj], 0, 0, 0);
        // step g+2 landed (g+3 may be in flight); bare barrier as in v3
        __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
        __builtin_amdgcn_s_barrier();
      }
      int tk = 0;
      if (wave_u == 0 && lane == 0)
        tk = lane_fetch_add(const_cast<int*>(p.count) + 4 + xcd, j_next < 0 ? 2 : 1);
      // ---- epilogue: the tile's last ring slot (step g-1) is consumed and is refilled only by the
      // next step's load; every wave's fragment reads of it complete before the staging writes
      // (LDS-only release fence, barrier).  acc[i][j][4q+c] of lane l is dW[row i*32 + l%32][col
      // j*32 + 8q + 4(l/32) + c]; each wave stages 32 rows x 64 columns (16-byte chunk c of row r at
      // chunk c ^ (r & 7)) and writes whole 128-byte row segments.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_s_barrier();
      char* wst = lds + ((g - 1) & (NSTAGE - 1)) * STAGE + wave * 4096;
      uint16_t* out = p.C + (int64_t)cur.e * p.Kd * p.N + (int64_t)cur.row0 * p.N + cur.col0;
      const uint32_t lo = (uint32_t)(wm * WTM + (lane >> 3)) * (uint32_t)p.N + (uint32_t)(wn * WTN + (lane & 7) * 8);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int jj = 0; jj < TN; ++jj)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
            *(bf16x4*)(wst + frow * 128 + (((4 * jj + gq) ^ (frow & 7)) << 4) + 8 * fhalf) =
                bf16x4{(__bf16)acc[i][jj][4 * gq], (__bf16)acc[i][jj][4 * gq + 1], (__bf16)acc[i][jj][4 * gq + 2],
                       (__bf16)acc[i][jj][4 * gq + 3]};
        __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int rloc = rr * 8 + (lane >> 3);
          const u32x4 v = *(const u32x4*)(wst + rloc * 128 + (((lane & 7) ^ (rloc & 7)) << 4));
          *(u32x4*)(out + lo + (uint32_t)(i * 32 + rr * 8) * (uint32_t)p.N) = v;
        }
        __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);  // reads done before the next block overwrites
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[i][jj][v] = 0.0f;
      if (wave_u == 0 && lane == 0) s_ticket = tk;
      __syncthreads();  // the staging slot and s_ticket
      const int t = s_ticket;  // rewritten only in the next epilogue
      const bool first = j_next < 0;
      if (first) j_next = nx + t;
      const int j_after = first ? nx + t + 1 : nx + t;  // tickets rise, so j_next invalid => j_after too
      j = j_next;
      if (!valid(j)) break;
      const bool chained = chain;
      if (first) nxt = decode(8 * j + xcd);
      cur = nxt;
      j_next = j_after;
      if (valid(j_next)) nxt = decode(8 * j_next + xcd);
      chain = valid(j_next) && cur.nk >= PD && nxt.nk >= PD;
      la = chain ? nxt : cur;
      if (!chained) {
        // every wave's re-reads have landed before the prologue refills the ring
        __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));
        __syncthreads();
        prologue();
      }
    }
    // the loads past the last tile land before the workgroup ends
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));
    __syncthreads();
  }
}

// ---- w4: one wave per SIMD (FWD / SWIGLU / DLHS, 256x256 tiles) ------------------------------------
// The v3 tile, ring, DMA layouts, fragment reads and MFMA order with 4 waves instead of 8: a wave
// owns a 128x128 quarter of the tile (16 accumulator blocks, which live in the AGPRs), so each
// SIMD runs one wave that interleaves its own fragment reads with its MFMAs instead of sharing the
// MFMA pipe with a second wave behind a per-stage barrier, and the fragment reads per stage drop
// from 96 KB to 64 KB per CU.  Every output element gets the MFMA sequence of gmm_v3_kernel
// (operands swapped, k in ring order), hence the same bits.  A tile with at most 128 rows of its
// group runs the thin form instead: the four waves split the 256 columns (128x64 wave tiles, the
// v3 wave tile) over the tile's ceil(rows/32) row blocks only, and the ring loads 128 A rows.
#ifndef MTX_W4_NSTAGE
#define MTX_W4_NSTAGE 4
#endif
namespace w4 {
// ring of NSTAGE 32 KB stages, PD = NSTAGE - 1 of them in flight ahead of the one computed
constexpr int NT = 256, BM = 256, BN = 256, NSTAGE = MTX_W4_NSTAGE, PD = NSTAGE - 1;
__device__ __forceinline__ int slot(int k) { return (NSTAGE & (NSTAGE - 1)) == 0 ? (k & (NSTAGE - 1)) : (k % NSTAGE); }
constexpr int A_BYTES = BM * v3::BKS * 2, STAGE = A_BYTES + BN * v3::BKS * 2;  // 16 + 16 KB

struct Tile {
  int e, r0, r1, n_tile;
  int piece, npieces, split_u;  // k-piece of a split tail tile (1 piece: whole tile)
  int queue;                    // tile queue (XCD range) the tile came from
};

// One tile with TM x TN 32x32 accumulator blocks per wave.  THIN: wave w owns the 32-column blocks
// of the tile's columns [64w, 64w + 64) (SwiGLU: gate block and its up block), rows 0 .. 32 TM.
template <int MODE, int EPI, int TM, int TN, bool THIN>
__device__ __forceinline__ void tile(const Args& p, char* lds, int* s_last, const Tile& t) {
  using v3::a_off;
  using v3::bn_off;
  using v3::BKS;
  constexpr int A_ROWS = THIN ? 128 : 256;
  constexpr int A_INSTR = A_ROWS * BKS * 2 / 1024 / 4;  // 1 KB load instructions per wave per stage
  constexpr int B_INSTR = 4;
  constexpr int LPS = A_INSTR + B_INSTR;
  constexpr bool B_T = (MODE == FWD);  // B stage stored [reduction][col] (transpose reads)
  static_assert(EPI != EPI_SWIGLU || TN % 2 == 0, "SwiGLU pairs gate/up blocks");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = THIN ? 0 : (wave >> 1);
  const int wn = THIN ? wave : (wave & 1);
  const int e = t.e, r0 = t.r0, r1 = t.r1, n_tile = t.n_tile, col0 = n_tile * BN;
  // tile-local column of the wave's 32-column block j; SwiGLU pairs gate block j with up block
  // j + TN/2 (64 tile columns further: the B stage holds, per 128 columns, 64 gate then 64 up)
  auto cbase = [&](int j) -> int {
    if constexpr (THIN) {
      if constexpr (EPI == EPI_SWIGLU) return (wn >> 1) * 128 + (wn & 1) * 32 + j * 64;
      return wn * 64 + j * 32;
    }
    return wn * 128 + j * 32;
  };

  const int nk_all = p.Kred / BKS;
  const int kb0 = t.piece * nk_all / t.npieces;
  const int nk = (t.piece + 1) * nk_all / t.npieces - kb0;

  // ---- per-lane global byte offsets of the ring loads at k-stage 0 (the v3 layouts) ---------
  uint32_t aoff[A_INSTR], boff[B_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) {
    const int seg = wave * A_INSTR + i;
    const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
    int gr = r0 + r;
    gr = gr < r1 ? gr : r1 - 1;  // rows past the group repeat its last row: never used, cache hits
    if (MODE == FWD && p.gather) gr = min(max(p.gather[gr], 0) / p.gather_div, p.gather_rows - 1);
    aoff[i] = ((uint32_t)gr * (uint32_t)p.Kred + (uint32_t)(c * 8)) * 2u;
  }
#pragma unroll
  for (int i = 0; i < B_INSTR; ++i) {
    const int seg = wave * B_INSTR + i;
    if constexpr (B_T) {
      const int k = seg * 2 + (lane >> 5), c = (lane & 31) ^ ((k & 3) << 2);
      const int tc = c * 8;
      int gc;
      if constexpr (EPI == EPI_SWIGLU) {
        const int w_ = tc >> 7, within = tc & 127;
        gc = (within >> 6) * p.I + n_tile * (BN / 2) + w_ * 64 + (within & 63);
      } else {
        gc = col0 + tc;
      }
      boff[i] = ((uint32_t)k * (uint32_t)p.N + (uint32_t)gc) * 2u;
    } else {
      const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
      boff[i] = ((uint32_t)(col0 + r) * (uint32_t)p.Kred + (uint32_t)(c * 8)) * 2u;
    }
  }
  const char* Ab = (const char*)p.A;
  const char* Bb = (const char*)(p.B + (int64_t)e * p.Kred * p.N);
  const int64_t b_step = B_T ? (int64_t)BKS * p.N * 2 : (int64_t)BKS * 2;
  const uint32_t lds_base = lds_addr(lds);
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  // stages past the end re-read the last one into a slot that is no longer read (branch-free)
  auto issue_stage = [&](int kt_) {
    const uint32_t st = lds_base + (uint32_t)(slot(kt_) * STAGE);
    const int kt = kb0 + min(kt_, nk - 1);
    const char* a = Ab + (int64_t)kt * (BKS * 2);
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) gload_lds16_s(a, aoff[i], st + (wave_u * A_INSTR + i) * 1024u);
    const char* b = Bb + (int64_t)kt * b_step;
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) gload_lds16_s(b, boff[i], st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
  };

  // ---- fragments ------------------------------------------------------------------------------
  bf16x8 fa[2][TM], fb[2][TN];
  const int frow = lane & 31, fhalf = lane >> 5;
  auto read_tr = [&](const char* region, int c0, int kk) -> bf16x8 {
    const int n = c0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int k = kk * 16 + 8 * fhalf + ((lane & 15) >> 2);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k, n >> 3) + (n & 7) * 2));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(region + bn_off(k + 4, n >> 3) + (n & 7) * 2));
    const s16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
  };
  auto read_frags = [&](int kt, int kk, int buf) {
    const char* st = lds + slot(kt) * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[buf][i] = *(const bf16x8*)(st + a_off(wm * 128 + i * 32 + frow, kk * 2 + fhalf));
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (B_T) fb[buf][j] = read_tr(st + A_BYTES, cbase(j), kk);
      else fb[buf][j] = *(const bf16x8*)(st + A_BYTES + a_off(cbase(j) + frow, kk * 2 + fhalf));
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // One load instruction of a ring stage: d < A_INSTR loads A, the rest B.
  auto issue_one = [&](int kt_, int d) {
    const uint32_t st = lds_base + (uint32_t)(slot(kt_) * STAGE);
    const int kt = kb0 + min(kt_, nk - 1);
    if (d < A_INSTR) {
      gload_lds16_s(Ab + (int64_t)kt * (BKS * 2), aoff[d], st + (wave_u * A_INSTR + d) * 1024u);
    } else {
      const int i = d - A_INSTR;
      gload_lds16_s(Bb + (int64_t)kt * b_step, boff[i], st + (uint32_t)A_BYTES + (wave_u * B_INSTR + i) * 1024u);
    }
  };
  // fragment slot r of a substep: r < TM reads A block r, else B block r - TM
  auto read_one = [&](int kt, int kk, int buf, int r) {
    const char* st = lds + slot(kt) * STAGE;
    if (r < TM) {
      fa[buf][r] = *(const bf16x8*)(st + a_off(wm * 128 + r * 32 + frow, kk * 2 + fhalf));
    } else {
      const int j = r - TM;
      if constexpr (B_T) fb[buf][j] = read_tr(st + A_BYTES, cbase(j), kk);
      else fb[buf][j] = *(const bf16x8*)(st + A_BYTES + a_off(cbase(j) + frow, kk * 2 + fhalf));
    }
  };

  // prologue: stages 0..PD-1 in flight, stage 0 landed and visible (stage 1, first read halfway
  // through stage 0, is waited for there)
#pragma unroll
  for (int s = 0; s < PD; ++s) issue_stage(s);
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 1)));
  __syncthreads();
  read_frags(0, 0, 0);
  // Each stage is 2 x S MFMA slots in a fixed order: slot q issues one MFMA, then one fragment read
  // of the other buffer (substep 1 of this stage during substep 0, substep 0 of the next stage
  // during substep 1), and the stage's LPS ring loads are spread evenly over the slots, so that the
  // single wave of the SIMD never stalls its MFMA issue on a burst of loads (+4-5 % on the Mixtral
  // shapes against issuing them together at the top of the stage).
  constexpr int S = TM * TN;
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int q = 0; q < 2 * S; ++q) {
      const int sub = q / S, qq = q % S;
      const int i = qq / TN, j = qq % TN;
      if (q == S && kt == 0) {
        // stage 1 landed (stage 2 and the first LPS/2 loads of stage 3 may be in flight) and
        // visible before its first fragment reads below
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS + LPS / 2));
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[sub][j], fa[sub][i], acc[i][j], 0, 0, 0);
      // fragment r goes in slot min(r, S-1): a substep with fewer MFMAs than fragments (TM = 1)
      // reads the rest in its last slot
#pragma unroll
      for (int r = 0; r < TM + TN; ++r) {
        if (min(r, S - 1) != qq) continue;
        if (sub == 0) read_one(kt, 1, 1, r);
        else read_one(kt + 1, 0, 0, r);  // visible since the last barrier (last step: an unused re-read)
      }
#pragma unroll
      for (int d = 0; d < LPS; ++d)
        if ((d * 2 * S) / LPS == q) issue_one(kt + PD, d);
    }
    __builtin_amdgcn_sched_barrier(0);
    // stage kt+2 landed before the barrier makes it visible; a bare s_barrier (the slot refilled
    // next held stage kt, whose fragments this iteration's MFMAs consumed)
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS * (PD - 2)));
    __builtin_amdgcn_s_barrier();
  }
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));  // no ring load may land after the ring is reused

  if (t.npieces > 1) {
    // split tail piece: as in gmm_v3_kernel (partials in piece order, summed by the last arrival)
    typedef __attribute__((ext_vector_type(4))) float f32x4;
    constexpr int64_t SLOT4 = kSplitSlotFloats / 4;
    static_assert(TM * TN * 4 * NT <= SLOT4, "split slot");
    const int xcd_e = t.queue;
    f32x4* part = (f32x4*)(p.split_part + (int64_t)(xcd_e * kSplitItems + t.split_u * t.npieces) * kSplitSlotFloats);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          part[t.piece * SLOT4 + ((i * TN + j) * 4 + g) * NT + tid] =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0)
      *s_last = __hip_atomic_fetch_add(p.split_cnt + xcd_e * kSplitMaxRem + t.split_u, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == t.npieces - 1;
    __syncthreads();
    if (!*s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#pragma unroll
    for (int s2 = 0; s2 < kSplitMaxS; ++s2) {
      if (s2 >= t.npieces) break;
      const f32x4* src = part + s2 * SLOT4;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 v = src[((i * TN + j) * 4 + g) * NT + tid];
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[i][j][4 * g + c] = (s2 == 0) ? v[c] : acc[i][j][4 * g + c] + v[c];
          }
    }
  }

  // ---- epilogue: acc[i][j][4g+q] of lane l is C[row i*32 + l%32][col cbase(j) + 8g + 4(l/32) + q];
  // the tile is staged in the idle ring as bf16 rows (16-byte chunk c of row r at c ^ (r & 15)) and
  // written back with 16 contiguous bytes per lane, whole 128-byte lines per row.
  constexpr int OCOLS = (EPI == EPI_SWIGLU) ? BN / 2 : BN;
  constexpr int OROW = OCOLS * 2, OCH = OROW / 16;
  static_assert(A_ROWS * OROW <= NSTAGE * STAGE, "staging fits the ring");
  auto stage4 = [&](int r, int col, bf16x4 v) {
    const int c = col >> 3;
    *(bf16x4*)(lds + r * OROW + ((c ^ (r & 15)) << 4) + (col & 7) * 2) = v;
  };
  __syncthreads();  // every wave is done with the ring
  {
    const int h4 = 4 * fhalf;
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN / 2; ++j) {
          const int cg = cbase(j), ocol = (cg >> 7) * 64 + (cg & 127);  // gate column -> output column
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x16& gt = acc[i][j];
            const f32x16& up = acc[i][j + TN / 2];
            stage4(wm * 128 + i * 32 + frow, ocol + 8 * g + h4,
                   bf16x4{(__bf16)swiglu_fast(gt[4 * g], up[4 * g]), (__bf16)swiglu_fast(gt[4 * g + 1], up[4 * g + 1]),
                          (__bf16)swiglu_fast(gt[4 * g + 2], up[4 * g + 2]),
                          (__bf16)swiglu_fast(gt[4 * g + 3], up[4 * g + 3])});
          }
        }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            stage4(wm * 128 + i * 32 + frow, cbase(j) + 8 * g + h4,
                   bf16x4{(__bf16)acc[i][j][4 * g], (__bf16)acc[i][j][4 * g + 1], (__bf16)acc[i][j][4 * g + 2],
                          (__bf16)acc[i][j][4 * g + 3]});
    }
  }
  __syncthreads();
  uint16_t* obase = p.C + ((EPI == EPI_SWIGLU) ? n_tile * (BN / 2) : col0);
  const int nrows = min(r1 - r0, A_ROWS);
  constexpr int RPI = 64 / OCH;  // rows per wave instruction
  for (int rr = wave * RPI + lane / OCH; rr < nrows; rr += NT / OCH) {
    const int c = lane % OCH;
    const u32x4 v = *(const u32x4*)(lds + rr * OROW + ((c ^ (rr & 15)) << 4));
    *(u32x4*)(obase + (int64_t)(r0 + rr) * p.ldc + c * 8) = v;
  }
}
}  // namespace w4

template <int MODE, int EPI>
__global__ __launch_bounds__(256, 1) void gmm_w4_kernel(Args p) {
  static_assert(MODE == FWD || MODE == DLHS, "w4 mode");
  __shared__ __attribute__((aligned(1024))) char lds[w4::NSTAGE * w4::STAGE];
  // two ints of workgroup state in the ring's last slot: the prologue leaves that slot alone (its
  // first load is issued after the prologue's barrier) and the split tail uses it after the k-loop
  int* s_misc = (int*)(lds + (w4::NSTAGE - 1) * w4::STAGE);
  constexpr int BN = w4::BN, NT = w4::NT;
  const int tid = threadIdx.x;
  // ---- which output tile.  The v3 order: queue x (the workgroups dispatched to XCD x, pid % 8)
  // owns the tile range [x*per, x*per + tx) -- gm m-tiles per scheduling group -- followed, when its
  // last round is sparse, by that round's tiles split into k-pieces (split tail).  Each XCD's first
  // ncu_x workgroups take their queue's first items in dispatch order; later workgroups take tickets
  // from their own queue and, once it is exhausted, from the other queues in turn, so that an XCD that
  // runs ahead finishes the others' tiles instead of idling at the end (the XCDs of one chip run the
  // same tile list 3-6 % apart).  Which workgroup computes an item does not change its result.
  w4::Tile t;
  t.piece = 0;
  t.npieces = 1;
  t.split_u = 0;
  const int nn = (EPI == EPI_SWIGLU) ? (p.I / (BN / 2)) : (p.N / BN);
  const int cnt = p.count[0];
  const int total = cnt * nn;
  const int pid = blockIdx.x;
  const int total8 = (total + 7) & ~7;
  const int xcd = pid & 7, q = pid >> 3, per = total8 >> 3;
  // items of queue x: nwhole whole tiles, then (S > 1) rem tiles in S pieces each
  auto queue_items = [&](int x, int& nwhole, int& S) -> int {
    const int tx = max(0, min(per, total - x * per));
    nwhole = tx;
    S = 1;
    if (EPI == EPI_STORE && p.split_on) {
      const int rem = tx % p.ncu_x;
      int S_ = (rem > 0 && rem <= kSplitMaxRem && 2 * rem <= p.ncu_x) ? min(kSplitMaxS, p.ncu_x / rem) : 1;
      S_ = min(S_, max(p.Kred / v3::BKS, 1));
      if (S_ > 1) {
        nwhole = tx - rem;
        S = S_;
        return nwhole + rem * S_;
      }
    }
    return tx;
  };
  int qx = xcd, nwhole, S;
  int nitems = queue_items(xcd, nwhole, S);
  int item = q;
  if (p.tickets != nullptr && q >= min(p.ncu_x, nitems)) {
    int* s_ticket = s_misc;
    if (tid == 0) {
      int got = -1, gq = 0;
      for (int k = 0; k < 8 && got < 0; ++k) {
        const int y = (xcd + k) & 7;
        int nw_, S_;
        const int ny = queue_items(y, nw_, S_), sy = min(p.ncu_x, ny);
        if (ny <= sy) continue;  // no items past the statically taken ones
        const int tk = __hip_atomic_fetch_add(p.tickets + y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + sy;
        if (tk < ny) {
          got = tk;
          gq = y;
        }
      }
      s_ticket[0] = got;
      s_ticket[1] = gq;
    }
    __syncthreads();
    item = s_ticket[0];
    qx = s_ticket[1];
    if (item < 0) return;
    nitems = queue_items(qx, nwhole, S);
  }
  if (item >= nitems) return;
  t.queue = qx;
  int lid;
  if (item < nwhole) {
    lid = qx * per + item;
  } else {
    t.split_u = (item - nwhole) / S;
    t.piece = (item - nwhole) % S;
    t.npieces = S;
    lid = qx * per + nwhole + t.split_u;
  }
  int first_m, gsz, n_first = 0, nspan = nn, l = lid;
  if (p.nsplit) {  // queue x: n-tiles [x*nb, (x+1)*nb) of every m-tile, per = cnt * nb
    const int nb = nn >> 3, x = lid / per;
    l = lid - x * per;
    n_first = x * nb;
    nspan = nb;
  }
  if (p.vgroup) {  // position l / nspan lies inside l's group
    const int g = p.tiles[l / nspan].pad;
    first_m = g >> 8;
    gsz = g & 255;
  } else {
    first_m = (l / (p.gm * nspan)) * p.gm;
    gsz = min(p.gm, cnt - first_m);
  }
  const int local = l - first_m * nspan;
  const MTile mt = p.tiles[first_m + local % gsz];
  t.e = mt.e;
  t.r0 = mt.r0;
  t.r1 = mt.r1;
  t.n_tile = n_first + local / gsz;
  if (t.e < 0) {  // rows past sum(group_sizes): zeros
    if (t.piece > 0) return;
    const int ncols = (EPI == EPI_SWIGLU) ? BN / 2 : BN;
    const int c0 = t.n_tile * ncols;
    for (int i = tid; i < w4::BM * ncols; i += NT) {
      const int r = t.r0 + i / ncols;
      if (r < t.r1) p.C[(int64_t)r * p.ldc + c0 + i % ncols] = 0;
    }
    return;
  }
  const int rows = t.r1 - t.r0;
  if (rows > 128) w4::tile<MODE, EPI, 4, 4, false>(p, lds, s_misc, t);
  else if (rows > 96) w4::tile<MODE, EPI, 4, 2, true>(p, lds, s_misc, t);
  else if (rows > 64) w4::tile<MODE, EPI, 3, 2, true>(p, lds, s_misc, t);
  else if (rows > 32) w4::tile<MODE, EPI, 2, 2, true>(p, lds, s_misc, t);
  else w4::tile<MODE, EPI, 1, 2, true>(p, lds, s_misc, t);
}

}  // namespace mf

// ---- host-side dispatch ----------------------------------------------------------------------
struct MfmaCfg {
  int BM, BN;
};

static int launch_build_tiles(const int32_t* gs, int64_t E, int64_t M, int BM, const GmmWs& w, hipStream_t st,
                              bool need_order = false, bool reset_split = false, int spread = 0, int align = 0,
                              int merge = 0) {
  hipLaunchKernelGGL(build_tiles_kernel, dim3(1), dim3(1024), 0, st, gs, (int)E, (int)M, BM, w.count, w.offsets,
                     w.order, w.tiles, need_order ? 1 : 0, reset_split ? w.split_cnt : (int*)nullptr, spread, align, merge);
  return check_launch();
}

// CUs per XCD of the current device (one resident 256-row workgroup per CU), cached per device.
static int cus_per_xcd() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = n / kSplitXcd;
  }
  return cache[dev];
}

// v3 configurations: 256x256 tiles with 8 waves (128x64 wave tiles) and a 4-deep ring (one
// workgroup per CU) for large groups; 128x256 tiles with 4 waves (64x128 wave tiles) and a
// 3-deep ring (72 KB, two workgroups per CU) for groups of about a hundred rows.
// Mean group size below which the 128-row configuration is used (0: always 256-row tiles,
// whose empty 32-row blocks skip their MFMAs, so each expert's weights stream once).
#ifndef MTX_GM_SMALL
#define MTX_GM_SMALL 1
#endif
// m-tiles an expert needs to be spread through the tile order (0: never)
#ifndef MTX_SPREAD_MIN
#define MTX_SPREAD_MIN 4
#endif
#ifndef MTX_V3_NSTAGE
#define MTX_V3_NSTAGE 4
#endif
#ifndef MTX_V3_WN
#define MTX_V3_WN 4
#endif
#ifndef MTX_V3_SMALL_MEAN
#define MTX_V3_SMALL_MEAN 0
#endif
template <int MODE, int EPI>
static int launch_v3(const mf::Args& a, int64_t grid, hipStream_t st) {
  if (grid <= 0) return MTX_OK;
  grid = round_up(grid, 8);
  hipLaunchKernelGGL((mf::gmm_v3_kernel<MODE, EPI, 2, MTX_V3_WN, 256, MTX_V3_NSTAGE>), dim3((unsigned)grid),
                     dim3(128 * MTX_V3_WN), 0, st, a);
  return check_launch();
}
#ifndef MTX_V3S_WM
#define MTX_V3S_WM 2
#endif
#ifndef MTX_V3S_WN
#define MTX_V3S_WN 2
#endif
#ifndef MTX_V3S_NST
#define MTX_V3S_NST 3
#endif
// Persistent plain-store kernel for reductions of 4 .. MTX_V4P_MAX_STAGES 32-k stages (0: never):
// one workgroup per CU, each walking its XCD's share of the tile list.  Measured against
// gmm_v3_kernel on the same box (E = 8, M = 16384, N = 4096): +36 % at Kred 512, +10 % at 1024,
// but -8 % at 2048 and -26 % at 4096, and -10 % / -19 % on the C5 dlhs / C3 down shapes (Kred
// 1536-2048).  vmcnt counts loads and stores in one in-order counter, so the next tile's first
// ring wait also waits for the previous tile's epilogue stores, which a short-lived v3 workgroup
// leaves draining behind it; that costs more than the saved ring fill once tiles are long.
#ifndef MTX_V4P_MAX_STAGES
#define MTX_V4P_MAX_STAGES 32
#endif
template <int MODE>
static int launch_v4p(const mf::Args& a, int64_t max_tiles, int ncu, hipStream_t st) {
  const int64_t grid = std::min(round_up(max_tiles, 8), (int64_t)kSplitXcd * ncu);
  if (grid <= 0) return MTX_OK;
  hipLaunchKernelGGL((mf::gmm_v4p_kernel<MODE>), dim3((unsigned)grid), dim3(512), 0, st, a);
  return check_launch();
}
// One-wave-per-SIMD kernel (gmm_w4_kernel) for the 256-row tile paths: bit 0 SwiGLU, bit 1 plain
// forward, bit 2 dlhs (0: gmm_v3_kernel everywhere); used when groups hold at least
// MTX_W4_MIN_MEAN rows on average.  Measured against gmm_v3_kernel (same bits): Mixtral shapes
// gate_up -3.4 to -5 %, down -2.4 to -3.5 %, Qwen3-shape dlhs -2 to -2.5 % time; DeepSeek-shape
// groups of ~128 rows +2 to +3 % (a 4-wave tile of 129-255 rows runs all its MFMAs, where v3 skips
// a wave pair's empty row blocks), hence the threshold.
#ifndef MTX_W4
#define MTX_W4 7
#endif
// gmm_w4_kernel: n-tiles split over the XCDs (bit 0 plain-store forward, bit 1 SwiGLU).  The eight
// XCDs then sweep the experts together, each over its eighth of the n-tiles, so an expert's A rows
// are fetched from HBM about once and re-read from the MALL, instead of once per group of n-tiles
// that an XCD sweeps: C2 down 1.73 -> 1.64 ms (three runs each).  The SwiGLU tiles (whose A, the
// token rows, fits the MALL anyway) measured equal, the C5 dlhs +2 % (Zipf loads), so those keep
// the contiguous XCD ranges.
#ifndef MTX_NSPLIT
#define MTX_NSPLIT 1
#endif
// m-tiles past an expert's last full scheduling group that stay in that group (gmm_w4_kernel)
#ifndef MTX_MERGE_REM
#define MTX_MERGE_REM 2
#endif
// 1: scheduling groups of the 256-row paths hold the m-tiles of one expert (build_tiles_kernel)
#ifndef MTX_ALIGN_GROUPS
#define MTX_ALIGN_GROUPS 1
#endif
#ifndef MTX_W4_MIN_MEAN
#define MTX_W4_MIN_MEAN 512
#endif
#ifndef MTX_W4_QUEUES
#define MTX_W4_QUEUES 1
#endif
template <int MODE, int EPI>
static int launch_w4(mf::Args a, int64_t grid, hipStream_t st) {
  if (grid <= 0) return MTX_OK;
  grid = round_up(grid, 8);
  const int ncu = cus_per_xcd();
  if (MTX_W4_QUEUES && ncu >= 1) {
    a.tickets = const_cast<int*>(a.count) + 4;  // zeroed by the tile-list kernel of this call
    a.ncu_x = ncu;
  }
  hipLaunchKernelGGL((mf::gmm_w4_kernel<MODE, EPI>), dim3((unsigned)grid), dim3(256), 0, st, a);
  return check_launch();
}
template <int MODE, int EPI>
static int launch_v3_small(const mf::Args& a, int64_t grid, hipStream_t st) {
  if (grid <= 0) return MTX_OK;
  grid = round_up(grid, 8);
  hipLaunchKernelGGL((mf::gmm_v3_kernel<MODE, EPI, MTX_V3S_WM, MTX_V3S_WN, 128, MTX_V3S_NST>), dim3((unsigned)grid),
                     dim3(64 * MTX_V3S_WM * MTX_V3S_WN), 0, st, a);
  return check_launch();
}

template <int BM, int BN, int WM, int WN, int MODE, int EPI>
static int launch_mfma(const mf::Args& a, int64_t grid, hipStream_t st) {
  if (grid <= 0) return MTX_OK;
  grid = round_up(grid, 8);  // the XCD remap inside the kernel assumes a multiple of 8
  hipLaunchKernelGGL((mf::gmm_mfma_kernel<BM, BN, WM, WN, MODE, EPI>), dim3((unsigned)grid), dim3(WM * WN * 64), 0,
                     st, a);
  return check_launch();
}

static int common_checks(int64_t M, int64_t E, void* ws, int64_t ws_bytes, int64_t BM) {
  if (M < 0 || M > INT32_MAX / 2 || E < 1 || E > 1024) return MTX_ERR_ARG;
  const int64_t need = gmm_ws_tiles_off(E) + gmm_max_tiles(M, E, BM) * (int64_t)sizeof(MTile);
  if (!ws || ws_bytes < need) return MTX_ERR_WORKSPACE;
  return MTX_OK;
}

// Smallest m-tile any path uses is 64 rows, so the workspace bound uses BM = 64.
static constexpr int kMinBM = 64;


// FWD / DLHS / SWIGLU driver. mode: 0 fwd, 1 dlhs, 2 swiglu.  tile_m (0, 128 or 256 rows per
// m-tile) and tile_group (0 or m-tiles per scheduling group) override the shape heuristics on the
// bf16 MFMA path; every configuration computes each output element with the same MFMA sequence.
// With gather (FWD / SWIGLU, bf16): A holds gather_rows rows and sorted row r reads A row
// gather[r] / gather_div; only the direct-to-LDS kernels take it (MTX_ERR_UNSUPPORTED otherwise).
static int gmm_driver(int mode, const void* x, const void* w, const int32_t* gs, int dtype, int64_t M, int64_t Kred,
                      int64_t Nout, int64_t I, int64_t E, void* out, void* ws, int64_t ws_bytes, hipStream_t st,
                      int tile_m = 0, int tile_group = 0, const int32_t* gather = nullptr, int64_t gather_div = 1,
                      int64_t gather_rows = 0) {
  if (dtype != MTX_F32 && dtype != MTX_BF16) return MTX_ERR_ARG;
  const bool gath = gather != nullptr;
  if (gath && (mode == 1 || gather_div < 1 || gather_div > INT32_MAX || gather_rows < 0 ||
               gather_rows > INT32_MAX / 2 || (gather_rows == 0 && M > 0)))
    return MTX_ERR_ARG;
  int rc = common_checks(M, E, ws, ws_bytes, kMinBM);
  if (rc != MTX_OK) return rc;
  if (Kred < 0 || Nout < 0 || Kred > INT32_MAX / 2 || Nout > INT32_MAX / 2) return MTX_ERR_ARG;
  if (M == 0 || Nout == 0) return MTX_OK;
  if (!x || !w || !gs || !out) return MTX_ERR_ARG;
  GmmWs wsp = gmm_ws(ws, M, E);
  const int64_t out_cols = (mode == 2) ? I : Nout;
  if (mode == 2 && Nout != 2 * I) return MTX_ERR_ARG;
  // bf16 MFMA eligibility
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0);
  if (gath && !(dtype == MTX_BF16 && aligned && Kred % mf::BK == 0 && Kred > 0)) return MTX_ERR_UNSUPPORTED;
  if (dtype == MTX_BF16 && aligned && Kred % mf::BK == 0 && Kred > 0) {
    mf::Args a;
    a.A = (const uint16_t*)x;
    a.B = (const uint16_t*)w;
    if (gath) {
      a.gather = gather;
      a.gather_div = (int)gather_div;
      a.gather_rows = (int)gather_rows;
    }
    a.C = (uint16_t*)out;
    a.count = wsp.count;
    a.offsets = wsp.offsets;
    a.order = wsp.order;
    a.tiles = wsp.tiles;
    a.M = (int)M;
    a.Kred = (int)Kred;
    a.N = (int)Nout;
    a.Kd = 0;
    a.ldc = (int)out_cols;
    a.I = (int)I;
    a.E = (int)E;
    // A tile group of gm m-tiles runs against a few n-tiles at a time on one XCD.  With several
    // m-tiles per expert, 8 balances the re-reads of x and W through L2; with about one m-tile
    // per expert (W is read once whatever the order) 1 keeps each x tile in L2 while all its
    // n-tiles run (C3 shapes: 6-7 % less time than 8).
    a.gm = tile_group > 0 ? tile_group : ((M / E) <= 256 ? MTX_GM_SMALL : 8);
    // tile shape: 256-row tiles when groups are large on average, else 128
    const bool v3ok = Kred % mf::v3::BKS == 0 && (gath ? gather_rows : M) * Kred * 2 < (int64_t(1) << 32) &&
                      Kred * Nout * 2 < (int64_t(1) << 32);
    const bool big_m = v3ok && (tile_m == 256 || (tile_m == 0 && (M / E) >= MTX_V3_SMALL_MEAN));
    if (gath && (!v3ok || !((mode == 2 && I % 128 == 0) || (mode == 0 && Nout % 256 == 0))))
      return MTX_ERR_UNSUPPORTED;
    // one m-tile per scheduling group: spread the m-tiles of experts with several of them
    const int spread = (a.gm == 1) ? MTX_SPREAD_MIN : 0;
    const bool w4 = big_m && (M / E) >= MTX_W4_MIN_MEAN;
    // groups of gm m-tiles that never mix experts (the 256-row paths, when the mean expert fills a
    // group: C2 -1 %; with Zipf loads, whose remainders then collect at the end of the list from
    // many experts, C5 dlhs ran 1-3 % slower): see build_tiles_kernel
    const int align = (MTX_ALIGN_GROUPS && a.gm > 1 && (M / E) >= 256 * a.gm) ? a.gm : 0;
    // gmm_w4_kernel SwiGLU: an expert's few m-tiles past its last full group join that group, so
    // that they read its weight strips from L2 beside their siblings (C2 gate_up -0.6 %, three
    // runs each; the plain-store tiles measured +0.5 % on C2 down: there the thin remainders at
    // the end of the list fill the last round's gaps)
    const int merge = (align > 0 && align + MTX_MERGE_REM <= 255 && M / 256 + E < (1 << 22)) ? MTX_MERGE_REM : 0;
    if (mode == 2 && I % 128 == 0) {
      if (big_m) {
        const bool use_w4 = (MTX_W4 & 1) && w4;
        a.vgroup = (use_w4 && merge > 0) ? 1 : 0;
        a.nsplit = ((MTX_NSPLIT & 2) && use_w4 && (I / 128) % 8 == 0) ? 1 : 0;
        rc = launch_build_tiles(gs, E, M, 256, wsp, st, false, false, spread, align, a.vgroup ? merge : 0);
        if (rc) return rc;
        if (use_w4) return launch_w4<mf::FWD, mf::EPI_SWIGLU>(a, gmm_max_tiles(M, E, 256) * (I / 128), st);
        return launch_v3<mf::FWD, mf::EPI_SWIGLU>(a, gmm_max_tiles(M, E, 256) * (I / 128), st);
      }
      rc = launch_build_tiles(gs, E, M, 128, wsp, st);
      if (rc) return rc;
      if (v3ok) return launch_v3_small<mf::FWD, mf::EPI_SWIGLU>(a, gmm_max_tiles(M, E, 128) * (I / 128), st);
      return launch_mfma<128, 256, 1, 2, mf::FWD, mf::EPI_SWIGLU>(a, gmm_max_tiles(M, E, 128) * (I / 128), st);
    }
    if (mode != 2 && Nout % 256 == 0) {
      const int64_t nks = Kred / mf::v3::BKS;
      const int ncu4 = cus_per_xcd();
      if (big_m && !gath && nks >= 4 && nks <= MTX_V4P_MAX_STAGES && ncu4 >= 1) {
        // short reductions: persistent workgroups, the ring running across tiles
        rc = launch_build_tiles(gs, E, M, 256, wsp, st, false, false, spread, align);
        if (rc) return rc;
        const int64_t tiles = gmm_max_tiles(M, E, 256) * (Nout / 256);
        return mode == 0 ? launch_v4p<mf::FWD>(a, tiles, ncu4, st) : launch_v4p<mf::DLHS>(a, tiles, ncu4, st);
      }
      if (big_m) {
        // split tail when the workspace carries the partials region (mtx_gmm_workspace_size)
        const int ncu = cus_per_xcd();
        const bool split = ws_bytes >= gmm_ws_split_off(M, E) + gmm_ws_split_bytes() && ncu >= 2 &&
                           ncu <= kSplitItems;
        if (split) {
          a.split_on = 1;
          a.split_cnt = wsp.split_cnt;
          a.split_part = wsp.split_part;
          a.ncu_x = ncu;
        }
        const bool use_w4 = ((mode == 0 && (MTX_W4 & 2)) || (mode == 1 && (MTX_W4 & 4))) && w4;
        a.nsplit = ((MTX_NSPLIT & 1) && use_w4 && mode == 0 && (Nout / 256) % 8 == 0) ? 1 : 0;
        rc = launch_build_tiles(gs, E, M, 256, wsp, st, false, split, spread, align);
        if (rc) return rc;
        // split pieces add at most ncu - rem < ncu workgroups per XCD
        const int64_t grid = round_up(gmm_max_tiles(M, E, 256) * (Nout / 256), 8) + (split ? 8 * (int64_t)ncu : 0);
        if (use_w4) return mode == 0 ? launch_w4<mf::FWD, mf::EPI_STORE>(a, grid, st)
                                     : launch_w4<mf::DLHS, mf::EPI_STORE>(a, grid, st);
        return mode == 0 ? launch_v3<mf::FWD, mf::EPI_STORE>(a, grid, st) : launch_v3<mf::DLHS, mf::EPI_STORE>(a, grid, st);
      }
      rc = launch_build_tiles(gs, E, M, 128, wsp, st);
      if (rc) return rc;
      const int64_t grid = gmm_max_tiles(M, E, 128) * (Nout / 256);
      if (v3ok)
        return mode == 0 ? launch_v3_small<mf::FWD, mf::EPI_STORE>(a, grid, st)
                         : launch_v3_small<mf::DLHS, mf::EPI_STORE>(a, grid, st);
      return mode == 0 ? launch_mfma<128, 256, 1, 2, mf::FWD, mf::EPI_STORE>(a, grid, st)
                       : launch_mfma<128, 256, 1, 2, mf::DLHS, mf::EPI_STORE>(a, grid, st);
    }
    if (mode != 2 && Nout % 128 == 0) {
      rc = launch_build_tiles(gs, E, M, 128, wsp, st);
      if (rc) return rc;
      const int64_t grid = gmm_max_tiles(M, E, 128) * (Nout / 128);
      return mode == 0 ? launch_mfma<128, 128, 2, 2, mf::FWD, mf::EPI_STORE>(a, grid, st)
                       : launch_mfma<128, 128, 2, 2, mf::DLHS, mf::EPI_STORE>(a, grid, st);
    }
  }
  // generic path (exact fp32 FMA; also bf16 shapes the MFMA tiling does not cover)
  if (gath) return MTX_ERR_UNSUPPORTED;
  rc = launch_build_tiles(gs, E, M, kMinBM, wsp, st);
  if (rc) return rc;
  const int64_t ntile_max = gmm_max_tiles(M, E, kMinBM);
  const int64_t gy = (mode == 2) ? ceil_div(I, 32) : ceil_div(Nout, 64);
  dim3 grid((unsigned)ntile_max, (unsigned)gy);
#define MTX_GEN(T, MD)                                                                                   \
  hipLaunchKernelGGL((gmm_generic_kernel<T, MD>), grid, dim3(256), 0, st, (const T*)x, (const T*)w, wsp.tiles, \
                     wsp.count, Kred, Nout, (T*)out)
  if (dtype == MTX_F32) {
    if (mode == 0) MTX_GEN(float, 0);
    else if (mode == 1) MTX_GEN(float, 1);
    else MTX_GEN(float, 2);
  } else {
    if (mode == 0) MTX_GEN(uint16_t, 0);
    else if (mode == 1) MTX_GEN(uint16_t, 1);
    else MTX_GEN(uint16_t, 2);
  }
#undef MTX_GEN
  return check_launch();
}

static int launch_swiglu(const void* h, int dtype, int64_t M, int64_t I, void* out, hipStream_t st) {
  if (M > 0 && swiglu_vec_ok(I, h, h, out)) {
    const int64_t vb = swiglu_vec_blocks(M, I);
#define MTX_SW(T, Q) hipLaunchKernelGGL((swiglu_vec_kernel<T, Q>), dim3(vb), dim3(256), 0, st, (const T*)h, M, I, (T*)out)
    if (dtype == MTX_F32) {
      if (swiglu_vec_narrow(M, I)) MTX_SW(float, uint32_t);
      else MTX_SW(float, uint64_t);
    } else {
      if (swiglu_vec_narrow(M, I)) MTX_SW(uint16_t, uint32_t);
      else MTX_SW(uint16_t, uint64_t);
    }
#undef MTX_SW
    return check_launch();
  }
  int64_t blocks = ceil_div(M * I, 256);
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) return MTX_OK;
  if (dtype == MTX_F32)
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3(blocks), dim3(256), 0, st, (const float*)h, M, I, (float*)out);
  else
    hipLaunchKernelGGL(swiglu_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t*)h, M, I,
                       (uint16_t*)out);
  return check_launch();
}

}  // namespace mtx

using namespace mtx;

// Tile lists, then the split-tail region (counters + fp32 partial tiles).  A workspace of at
// least the tile-list part (common_checks) is accepted; the split tail runs only with the full
// size returned here.
extern "C" int64_t mtx_gmm_workspace_size(int64_t M, int64_t E) {
  if (M < 0 || E < 1) return -1;
  return gmm_ws_split_off(M, E) + gmm_ws_split_bytes();
}

extern "C" int mtx_gmm(const void* x, const void* w, const int32_t* group_sizes, int dtype, int64_t M, int64_t Kin,
                       int64_t Kout, int64_t E, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  return gmm_driver(0, x, w, group_sizes, dtype, M, Kin, Kout, 0, E, out, workspace, workspace_bytes,
                    (hipStream_t)stream);
}

extern "C" int mtx_gmm_dlhs(const void* g, const void* w, const int32_t* group_sizes, int dtype, int64_t M,
                            int64_t Kin, int64_t Kout, int64_t E, void* dx, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  // reduction over Kout, output columns Kin
  return gmm_driver(1, g, w, group_sizes, dtype, M, Kout, Kin, 0, E, dx, workspace, workspace_bytes,
                    (hipStream_t)stream);
}

extern "C" int mtx_gmm_swiglu(const void* x, const void* w, const int32_t* group_sizes, int dtype, int64_t M,
                              int64_t Kin, int64_t I, int64_t E, void* out, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  if (I < 0) return MTX_ERR_ARG;
  const int rc = gmm_driver(2, x, w, group_sizes, dtype, M, Kin, 2 * I, I, E, out, workspace, workspace_bytes,
                            (hipStream_t)stream);
  return rc;
}

extern "C" int mtx_gmm_tiled(int op, const void* x, const void* w, const int32_t* group_sizes, int dtype, int64_t M,
                             int64_t Kin, int64_t Kout, int64_t E, int64_t tile_m, int64_t tile_group, void* out,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  if (tile_m != 0 && tile_m != 128 && tile_m != 256) return MTX_ERR_ARG;
  if (tile_group < 0 || tile_group > 64) return MTX_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int tm = (int)tile_m, tg = (int)tile_group;
  switch (op) {
    case MTX_GMM_OP_FWD:
      return gmm_driver(0, x, w, group_sizes, dtype, M, Kin, Kout, 0, E, out, workspace, workspace_bytes, st, tm, tg);
    case MTX_GMM_OP_DLHS:
      return gmm_driver(1, x, w, group_sizes, dtype, M, Kout, Kin, 0, E, out, workspace, workspace_bytes, st, tm, tg);
    case MTX_GMM_OP_SWIGLU:
      if (Kout < 0) return MTX_ERR_ARG;
      return gmm_driver(2, x, w, group_sizes, dtype, M, Kin, 2 * Kout, Kout, E, out, workspace, workspace_bytes, st,
                        tm, tg);
    default:
      return MTX_ERR_ARG;
  }
}

extern "C" int mtx_gmm_gathered(int op, const void* x, int64_t x_rows, const int32_t* row_index, int64_t index_div,
                                const void* w, const int32_t* group_sizes, int dtype, int64_t M, int64_t Kin,
                                int64_t Kout, int64_t E, int64_t tile_m, int64_t tile_group, void* out,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  if (!row_index && M > 0) return MTX_ERR_ARG;
  if (tile_m != 0 && tile_m != 128 && tile_m != 256) return MTX_ERR_ARG;
  if (tile_group < 0 || tile_group > 64) return MTX_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int tm = (int)tile_m, tg = (int)tile_group;
  switch (op) {
    case MTX_GMM_OP_FWD:
      return gmm_driver(0, x, w, group_sizes, dtype, M, Kin, Kout, 0, E, out, workspace, workspace_bytes, st, tm, tg,
                        row_index, index_div, x_rows);
    case MTX_GMM_OP_SWIGLU:
      if (Kout < 0) return MTX_ERR_ARG;
      return gmm_driver(2, x, w, group_sizes, dtype, M, Kin, 2 * Kout, Kout, E, out, workspace, workspace_bytes, st,
                        tm, tg, row_index, index_div, x_rows);
    default:
      return MTX_ERR_ARG;
  }
}

extern "C" int mtx_swiglu(const void* h, int dtype, int64_t M, int64_t I, void* out, void* stream) {
  if (M < 0 || I < 0 || (dtype != MTX_F32 && dtype != MTX_BF16)) return MTX_ERR_ARG;
  if (M == 0 || I == 0) return MTX_OK;
  if (!h || !out) return MTX_ERR_ARG;
  return launch_swiglu(h, dtype, M, I, out, (hipStream_t)stream);
}

#ifndef MTX_TGMM_V4P
#define MTX_TGMM_V4P 1
#endif
extern "C" int mtx_tgmm(const void* x, const void* g, const int32_t* group_sizes, int dtype, int64_t M, int64_t K,
                        int64_t N, int64_t E, void* dw, void* workspace, int64_t workspace_bytes, void* stream) {
  if (dtype != MTX_F32 && dtype != MTX_BF16) return MTX_ERR_ARG;
  int rc = common_checks(M, E, workspace, workspace_bytes, kMinBM);
  if (rc != MTX_OK) return rc;
  if (K < 0 || N < 0 || K > INT32_MAX / 2 || N > INT32_MAX / 2) return MTX_ERR_ARG;
  if (K == 0 || N == 0) return MTX_OK;
  if (!dw || !group_sizes || (M > 0 && (!x || !g))) return MTX_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  GmmWs wsp = gmm_ws(workspace, M, E);
  rc = launch_build_tiles(group_sizes, E, M, kMinBM, wsp, st, true);
  if (rc) return rc;
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)g % 16 == 0);
  if (dtype == MTX_BF16 && aligned && K % 128 == 0 && N % 128 == 0 && M > 0) {
    mf::Args a;
    a.A = (const uint16_t*)x;
    a.B = (const uint16_t*)g;
    a.C = (uint16_t*)dw;
    a.count = wsp.count;
    a.offsets = wsp.offsets;
    a.order = wsp.order;
    a.tiles = wsp.tiles;
    a.M = (int)M;
    a.Kred = 0;
    a.N = (int)N;
    a.Kd = (int)K;
    a.ldc = (int)N;
    a.I = 0;
    a.E = (int)E;
    a.gm = 8;
    if (K % 256 == 0 && N % 256 == 0 && M * K * 2 < (int64_t(1) << 32) && M * N * 2 < (int64_t(1) << 32)) {
      // XCD rectangles of each expert's tile grid: xa x xb = 8, xa | K/256, xb | N/256, fewest
      // blocks per XCD
      const int nr = (int)(K / 256), nc = (int)(N / 256);
      int best = 1 << 30;
      for (int xa = 1; xa <= 8; xa *= 2) {
        const int xb = 8 / xa;
        if (nr % xa || nc % xb || nr / xa + nc / xb >= best) continue;
        best = nr / xa + nc / xb;
        a.xa = xa;
        a.xb = xb;
      }
      // with 8 or more tiles per CU: persistent workgroups, the ring running across tiles
      const int64_t tiles = E * (K / 256) * (N / 256);
      const int ncu4 = cus_per_xcd();
      if (MTX_TGMM_V4P && ncu4 >= 1 && tiles >= (int64_t)8 * kSplitXcd * ncu4) {
        hipLaunchKernelGGL(mf::tgmm_v4p_kernel, dim3((unsigned)(kSplitXcd * ncu4)), dim3(512), 0, st, a);
        return check_launch();
      }
      return launch_v3<mf::TGMM, mf::EPI_STORE>(a, tiles, st);
    }
    if (K % 256 == 0 && N % 256 == 0) {
      const int64_t grid = round_up(E * (K / 256) * (N / 256), 8);
      return launch_mfma<256, 256, 2, 2, mf::TGMM, mf::EPI_STORE>(a, grid, st);
    }
    const int64_t grid = round_up(E * (K / 128) * (N / 128), 8);
    return launch_mfma<128, 128, 2, 2, mf::TGMM, mf::EPI_STORE>(a, grid, st);
  }
  dim3 grid((unsigned)E, (unsigned)ceil_div(K, 64), (unsigned)ceil_div(N, 64));
  if (dtype == MTX_F32)
    hipLaunchKernelGGL(tgmm_generic_kernel<float>, grid, dim3(256), 0, st, (const float*)x, (const float*)g,
                       wsp.offsets, K, N, (float*)dw);
  else
    hipLaunchKernelGGL(tgmm_generic_kernel<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)g, wsp.offsets, K, N, (uint16_t*)dw);
  return check_launch();
}

extern "C" int mtx_swiglu_bwd(const void* h, const void* dy, int dtype, int64_t M, int64_t I, void* dh, void* stream) {
  if (M < 0 || I < 0 || (dtype != MTX_F32 && dtype != MTX_BF16)) return MTX_ERR_ARG;
  if (M == 0 || I == 0) return MTX_OK;
  if (!h || !dy || !dh) return MTX_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (swiglu_vec_ok(I, h, dy, dh)) {
    const int64_t vb = swiglu_vec_blocks(M, I);
#define MTX_SW(T, Q)                                                                                          \
  hipLaunchKernelGGL((swiglu_bwd_vec_kernel<T, Q>), dim3(vb), dim3(256), 0, st, (const T*)h, (const T*)dy, M, I, \
                     (T*)dh)
    if (dtype == MTX_F32) {
      if (swiglu_vec_narrow(M, I)) MTX_SW(float, uint32_t);
      else MTX_SW(float, uint64_t);
    } else {
      if (swiglu_vec_narrow(M, I)) MTX_SW(uint16_t, uint32_t);
      else MTX_SW(uint16_t, uint64_t);
    }
#undef MTX_SW
    return check_launch();
  }
  int64_t blocks = ceil_div(M * I, 256);
  if (blocks > 65536) blocks = 65536;
  if (dtype == MTX_F32)
    hipLaunchKernelGGL(swiglu_bwd_kernel<float>, dim3(blocks), dim3(256), 0, st, (const float*)h, (const float*)dy, M,
                       I, (float*)dh);
  else
    hipLaunchKernelGGL(swiglu_bwd_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t*)h,
                       (const uint16_t*)dy, M, I, (uint16_t*)dh);
  return check_launch();
}

// ---- mtx_gmm_tiled without a caller workspace ---------------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture, serving loops):
// the tile lists live in `scratch`, a file-scope device array of kNoAllocScratchBytes, one copy
// per device, held until the process ends.  Its address on each device comes from
// hipGetSymbolAddress on the first call with that device current and is passed to the kernels like
// a workspace; the symbol itself is never handed to device code from the host.  The array holds
// no split-tail partials, so every tile runs whole (the results equal mtx_gmm_tiled's with a
// tile-list-only workspace, bit for bit).  The tile-list kernel of each call rewrites everything
// the GEMM reads from the array, so no clearing is needed between calls; calls that overlap on
// one device (concurrent streams or threads) race on the array.
namespace mtx {
constexpr int64_t kNoAllocMaxM = MTX_GMM_NOALLOC_MAX_ROWS;
constexpr int64_t kNoAllocMaxE = MTX_GMM_NOALLOC_MAX_EXPERTS;
constexpr int64_t kNoAllocScratchBytes =
    ((48 + 2 * kNoAllocMaxE + 1) * 4 + 255) / 256 * 256 + (kNoAllocMaxM / kMinBM + kNoAllocMaxE + 1) * 16;
static_assert(sizeof(MTile) == 16, "tile record size");
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {nullptr};

// The device address of `scratch` on the current device (looked up once per device).
static int scratch_ptr_current(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    g_last_hip_error = (int)e;
    return MTX_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return MTX_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      g_last_hip_error = (int)e;
      return MTX_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MTX_OK;
}
}  // namespace mtx

extern "C" int mtx_gmm_tiled_noalloc(int op, const void* x, const void* w, const int32_t* group_sizes, int dtype,
                                     int64_t M, int64_t Kin, int64_t Kout, int64_t E, int64_t tile_m,
                                     int64_t tile_group, void* out, void* stream) {
  if (M < 0 || E < 1) return MTX_ERR_ARG;
  if (M > kNoAllocMaxM || E > kNoAllocMaxE) return MTX_ERR_UNSUPPORTED;  // beyond the scratch array
  void* ws = nullptr;
  const int rc = scratch_ptr_current(&ws);
  if (rc != MTX_OK) return rc;
  return mtx_gmm_tiled(op, x, w, group_sizes, dtype, M, Kin, Kout, E, tile_m, tile_group, out, ws,
                       kNoAllocScratchBytes, stream);
}
