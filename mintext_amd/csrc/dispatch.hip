// Token dispatch (route) and combine (unroute) for the MoE layer on gfx950.
//
// route (bzantium/mintext mintext/kernels/moe_dispatch.py:47-81) is a stable argsort of
// ravel(topk_indices) by expert id, a row gather x[p // K] in that order and a bincount.
// Here the argsort is a stable counting sort, with no comparison sort and no atomics in
// the ranking, in two launches:
//   1. route_count   : one workgroup per chunk of the flat index array builds an LDS
//                      histogram over E+1 buckets (bucket E = ids outside [0,E)), stored
//                      bucket-major [bucket][chunk].
//   2. route_scatter : each chunk first derives its own offsets from the whole count table
//                      (bucket b's offset = all ids of buckets < b + ids of bucket b in
//                      earlier chunks: row sums, a scan over the buckets, a partial row
//                      sum), then ranks its elements in flat order; within a wave the rank
//                      is a ballot "multisplit" (log2(E+1) ballots build the mask of lanes
//                      with an equal key, rank = popcount of the lower lanes), across waves
//                      per-wave counts in LDS, across sub-tiles a running LDS base.
//   3. gather_rows   : one wave per output row, 16-byte vector copies.
// unroute (moe_dispatch.py:84-111) inverts the permutation (scatter of j to perm[j]) and
// combines out[n] = sum_k w[n,k] * Y[inv[n*K+k]] in f32 with k ascending, one wave per token.
#include <type_traits>
#include "common.h"

namespace mtx {

int g_last_hip_error = 0;

static constexpr int kRouteThreads = 256;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

struct RoutePlan {
  int64_t M;
  int nb;      // number of buckets = E + 1
  int nchunks;
  int cstride;  // count-table row length: nchunks rounded up to 4 (the pad columns hold 0)
  int64_t chunk;
  int64_t ws_counts;  // bytes
};

// About 1024 ids per chunk, at most 256 chunks, and at most 16384 entries in the count table,
// which every scatter workgroup reads whole.
static RoutePlan route_plan(int64_t N, int64_t K, int64_t E) {
  RoutePlan p;
  p.M = N * K;
  p.nb = (int)E + 1;
  int64_t nch = ceil_div(p.M, 1024);
  const int64_t cap = 16384 / p.nb;
  if (nch > cap) nch = cap;
  if (nch > 256) nch = 256;
  if (nch < 1) nch = 1;
  p.chunk = round_up(ceil_div(p.M > 0 ? p.M : 1, nch), kRouteThreads);
  p.nchunks = (int)ceil_div(p.M > 0 ? p.M : 1, p.chunk);
  p.cstride = (int)round_up(p.nchunks, 4);
  p.ws_counts = round_up((int64_t)p.cstride * p.nb * 4, 256);
  return p;
}

__device__ __forceinline__ int route_key(const int32_t* idx, int64_t p, int E) {
  const int v = idx[p];
  return (v < 0 || v >= E) ? E : v;
}

// counts[b * cstride + c] = ids of chunk c in bucket b; workgroup 0 also zeroes the pad columns.
__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(
    const int32_t* __restrict__ idx, int64_t M, int E, int nb, int64_t chunk, int nchunks, int cstride,
    int32_t* __restrict__ counts) {
  extern __shared__ int hist[];
  for (int b = threadIdx.x; b < nb; b += blockDim.x) hist[b] = 0;
  __syncthreads();
  const int64_t start = (int64_t)blockIdx.x * chunk;
  const int64_t end = min(start + chunk, M);
  constexpr int U = 8;  // ids loaded per lane before their atomics
  for (int64_t p0 = start + threadIdx.x; p0 < end; p0 += (int64_t)U * kRouteThreads) {
    int k[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t p = p0 + (int64_t)u * kRouteThreads;
      k[u] = p < end ? route_key(idx, p, E) : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k[u] >= 0) atomicAdd(&hist[k[u]], 1);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < nb; b += blockDim.x)
    counts[(int64_t)b * cstride + blockIdx.x] = hist[b];
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < nb * (cstride - nchunks); i += blockDim.x)
      counts[(int64_t)(i / (cstride - nchunks)) * cstride + nchunks + i % (cstride - nchunks)] = 0;
}

// Few experts and few ids: the whole stable counting sort in one workgroup of 1024 threads
// (nb = E+1 <= NB).  The keys are first staged in LDS as bytes with coalesced loads (16 in
// flight per thread).  Wave w owns the contiguous ids [w*C, (w+1)*C), C a multiple of 64, and
// walks them 64 at a time, lane l on id j0+l: a ballot per bucket counts the bucket's ids of the
// round (pass 1) and ranks each id among them (pass 2, mbcnt).  Exclusive scans over the waves
// (per bucket) and over the buckets give the bases, so positions follow the flat order within a
// bucket: the stable argsort's order.  Lanes on consecutive ids keep the inverse stores coalesced
// and the permutation stores in at most nb runs per instruction.
// Cost: about 7 lane-operations per id and bucket on one CU (64 lanes a clock), i.e. about
// M*nb/9 clocks: below the count/scan/scatter kernels' fixed cost only for small M*nb.
template <int NB>
__global__ __launch_bounds__(1024) void route_small_kernel(const int32_t* __restrict__ idx, int M, int E,
                                                           int32_t* __restrict__ perm, int32_t* __restrict__ inv,
                                                           int32_t* __restrict__ group_sizes) {
  extern __shared__ uint8_t kb[];  // [M] keys
  __shared__ int wtot[16][NB];
  __shared__ int bbase[NB];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int nb = E + 1;
  constexpr int U = 16;
  for (int j0 = t; j0 < M; j0 += 1024 * U) {
    int k[U];
#pragma unroll
    for (int u = 0; u < U; ++u) k[u] = route_key(idx, min(j0 + u * 1024, M - 1), E);  // in bounds
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j0 + u * 1024 < M) kb[j0 + u * 1024] = (uint8_t)k[u];
  }
  __syncthreads();
  const int C = ((M + 1023) >> 10) << 6;
  const int c0 = min(w * C, M), c1 = min(c0 + C, M);
  int tot[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) tot[b] = 0;
  for (int j0 = c0; j0 < c1; j0 += 64) {  // wave-uniform bounds: every lane takes part in the ballots
    const int j = j0 + lane;
    const int k = (j < c1) ? (int)kb[j] : NB;  // NB matches no bucket
#pragma unroll
    for (int b = 0; b < NB; ++b) tot[b] += __popcll(__ballot(k == b));
  }
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) wtot[w][b] = tot[b];
  }
  __syncthreads();
  if (t < nb) {  // bucket t: exclusive scan over the waves, and its total
    int run = 0;
    for (int ww = 0; ww < 16; ++ww) {
      const int x = wtot[ww][t];
      wtot[ww][t] = run;
      run += x;
    }
    bbase[t] = run;
  }
  __syncthreads();
  if (t == 0) {  // bucket bases in bucket order (the invalid-id bucket E last)
    int run = 0;
    for (int b = 0; b < nb; ++b) {
      const int x = bbase[b];
      if (b < E) group_sizes[b] = x;
      bbase[b] = run;
      run += x;
    }
  }
  __syncthreads();
  int base[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) base[b] = (b < nb) ? bbase[b] + wtot[w][b] : 0;
  for (int j0 = c0; j0 < c1; j0 += 64) {
    const int j = j0 + lane;
    const int k = (j < c1) ? (int)kb[j] : NB;
    int p = 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint64_t m = __ballot(k == b);
      const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (k == b) p = base[b] + below;
      base[b] += __popcll(m);
    }
    if (j < c1) {
      perm[p] = j;
      if (inv) inv[j] = p;
    }
  }
}

// Chunk c's offsets from the bucket-major count table (every workgroup reads the whole table,
// at most 16384 entries, as 16-byte units): row sums R[b] and the sums P[b] over the chunks
// before c, an exclusive scan of R over the buckets (thread t scans rows 4t..4t+3), run[b] =
// scan[b] + P[b]; workgroup 0 writes group_sizes = R.  Then the elements are ranked in flat
// order and scattered.
__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(
    const int32_t* __restrict__ idx, int64_t M, int E, int nb, int nbits, int64_t chunk, int cstride,
    const int32_t* __restrict__ counts, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ group_sizes) {
  extern __shared__ int sh[];
  const int nu = nb * (cstride >> 2);  // 16-byte units of the count table (<= 4096)
  int* run = sh;               // [nb]
  int* wcnt = sh + nb;         // [4][nb]
  int* rsum = sh + 5 * nb;     // [nb]
  int* ur = sh + 6 * nb;       // [nu] unit sums
  int* up = sh + 6 * nb + nu;  // [nu] unit sums over the chunks before this one
  __shared__ int wtot[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = blockIdx.x;
  // row sums and partial row sums: unit sums first (eight loads in flight per lane), then one
  // thread per row adds its units
  {
    const u32x4* tab = (const u32x4*)counts;
    const int upr = cstride >> 2;
    constexpr int U = 8;
    for (int i0 = tid; i0 < nu; i0 += kRouteThreads * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = tab[min(i0 + u * kRouteThreads, nu - 1)];  // in bounds
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kRouteThreads;
        if (i < nu) {
          const int c0 = 4 * (i % upr);
          int r = 0, pre = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            r += (int)v[u][k];
            pre += (c0 + k < c) ? (int)v[u][k] : 0;
          }
          ur[i] = r;
          up[i] = pre;
        }
      }
    }
    __syncthreads();
    for (int b = tid; b < nb; b += kRouteThreads) {
      int r = 0, pre = 0;
      for (int q = 0; q < upr; ++q) {
        r += ur[b * upr + q];
        pre += up[b * upr + q];
      }
      rsum[b] = r;
      run[b] = pre;
    }
  }
  __syncthreads();
  // exclusive scan of rsum over the buckets (nb <= 1024: four rows per thread)
  int loc[4], tsum = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = 4 * tid + k;
    loc[k] = (b < nb) ? rsum[b] : 0;
    tsum += loc[k];
  }
  int incl = tsum;
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) wtot[w] = incl;
  __syncthreads();
  int base = incl - tsum;
  for (int ww = 0; ww < w; ++ww) base += wtot[ww];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = 4 * tid + k;
    if (b < nb) {
      run[b] += base;
      if (c == 0 && b < E) group_sizes[b] = loc[k];
    }
    base += loc[k];
  }
  // Ranking in flat order, 256 ids per step: within a wave a ballot multisplit, across the four
  // waves per-wave counts in LDS, across steps the running bases run[]; the ids of U steps are
  // loaded before their ranking.
  const int64_t start = (int64_t)c * chunk;
  const int64_t end = min(start + chunk, M);
  const unsigned long long lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  constexpr int U = 8;
  int kreg[U];
  for (int64_t sb = start; sb < end; sb += kRouteThreads) {
    const int u = (int)(((sb - start) / kRouteThreads) % U);
    if (u == 0) {
#pragma unroll
      for (int v = 0; v < U; ++v) {
        const int64_t p = sb + (int64_t)v * kRouteThreads + tid;
        kreg[v] = p < end ? route_key(idx, p, E) : 0;
      }
    }
    for (int b = tid; b < 4 * nb; b += blockDim.x) wcnt[b] = 0;
    __syncthreads();
    const int64_t p = sb + tid;
    const bool valid = p < end;
    int key = 0;
#pragma unroll
    for (int v = 0; v < U; ++v)
      if (v == u) key = kreg[v];
    unsigned long long m = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (key >> bit) & 1;
      const unsigned long long bb = __ballot(on);
      m &= on ? bb : ~bb;
    }
    const int rank = __popcll(m & lt);
    const int cnt = __popcll(m);
    if (valid && rank == 0) wcnt[w * nb + key] = cnt;
    __syncthreads();
    if (valid) {
      int pos = run[key] + rank;
      for (int ww = 0; ww < w; ++ww) pos += wcnt[ww * nb + key];
      perm[pos] = (int32_t)p;
      if (inv) inv[p] = pos;
    }
    __syncthreads();
    if (valid && rank == 0) atomicAdd(&run[key], cnt);
    __syncthreads();
  }
}

// out[j] = src[index[j] / div] for rows of `row_bytes` bytes; VT is the copy unit.
template <typename VT>
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const char* __restrict__ src, int64_t src_rows, int64_t row_bytes,
    const int32_t* __restrict__ index, int64_t rows, int64_t div, char* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = row_bytes / (int64_t)sizeof(VT);
  const int64_t wave_id = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t j = wave_id; j < rows; j += nwaves) {
    const int64_t p = index[j];
    const int64_t r = (p >= 0) ? p / div : -1;
    VT* o = (VT*)(out + j * row_bytes);
    if (r < 0 || r >= src_rows) {
      VT z;
      memset(&z, 0, sizeof(VT));
      for (int64_t c = lane; c < nvec; c += 64) o[c] = z;
      continue;
    }
    const VT* s = (const VT*)(src + r * row_bytes);
    int64_t c = lane;
    for (; c + 192 < nvec; c += 256) {
      const VT a0 = s[c], a1 = s[c + 64], a2 = s[c + 128], a3 = s[c + 192];
      o[c] = a0; o[c + 64] = a1; o[c + 128] = a2; o[c + 192] = a3;
    }
    for (; c < nvec; c += 64) o[c] = s[c];
  }
}

// 16-byte-aligned rows: out[j] = src[index[j] / div] as a flat list of 16-byte items (row j,
// chunk c); each thread moves UNR items per step with all loads issued before the stores, so
// short rows (fp8 scale rows of 64 bytes) keep every lane busy and long rows keep UNR loads in
// flight per lane.
template <int UNR>
__global__ __launch_bounds__(256) void gather_chunks_kernel(
    const char* __restrict__ src, int64_t src_rows, int64_t cpr, int cpr_shift,
    const int32_t* __restrict__ index, int64_t rows, int64_t div, char* __restrict__ out) {
  const int64_t total = rows * cpr;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; base < total; base += stride * UNR) {
    u32x4 v[UNR];
    int64_t dst[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t it = base + u * stride;
      dst[u] = -1;
      if (it < total) {
        const int64_t j = cpr_shift >= 0 ? (it >> cpr_shift) : it / cpr;
        const int64_t c = it - j * cpr;
        const int p = index[j];
        const int64_t r = (p >= 0) ? (int64_t)(p / (int)div) : -1;
        dst[u] = it;
        if (r >= 0 && r < src_rows) v[u] = ((const u32x4*)src)[r * cpr + c];
        else v[u] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
      if (dst[u] >= 0) ((u32x4*)out)[dst[u]] = v[u];
  }
}

// Dispatch in token order (moe_dispatch.py:67,76 without the materialised repeat): token row n
// is read once and written to its K sorted positions, out[inv[n*K+k]] = src[n].  Items are
// 16-byte chunks (n, c) of the data rows (cpr chunks per row) followed by those of the optional
// scale rows (spr chunks per row), so both matrices move in one launch.  Each thread loads UNR
// items before storing any of them (UNR loads and UNR*K stores in flight per lane).
template <int UNR>
__global__ __launch_bounds__(256) void dispatch_rows_kernel(
    const u32x4* __restrict__ src, int64_t N, int64_t cpr, int cpr_shift, const u32x4* __restrict__ ssrc,
    int64_t spr, const int32_t* __restrict__ inv, int K, u32x4* __restrict__ out, u32x4* __restrict__ sout) {
  const int64_t nd = N * cpr;
  const int64_t total = nd + N * spr;
  const int64_t M = N * (int64_t)K;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; base < total; base += stride * UNR) {
    u32x4 v[UNR];
    int64_t n[UNR], c[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t it = base + u * stride;
      n[u] = -1;
      if (it < nd) {
        n[u] = cpr_shift >= 0 ? (it >> cpr_shift) : it / cpr;
        c[u] = it - n[u] * cpr;
        v[u] = src[it];
      } else if (it < total) {
        const int64_t i2 = it - nd;
        n[u] = i2 / spr;
        c[u] = i2 - n[u] * spr;
        v[u] = ssrc[i2];
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      if (n[u] < 0) continue;
      const bool data = (base + u * stride) < nd;
      for (int k = 0; k < K; ++k) {
        const int64_t j = inv[n[u] * K + k];
        if (j < 0 || j >= M) continue;
        if (data) out[j * cpr + c[u]] = v[u];
        else sout[j * spr + c[u]] = v[u];
      }
    }
  }
}

// Quantise-and-dispatch in token order: the 1x128 e4m3 quantiser of quant_rows_kernel (same
// group maximum, scale = amax / 448 or 1 when the group is all zeros, codes of v / scale) fused
// with the row dispatch, so each token row is read once in its compute dtype and only its fp8
// codes and scales are written, to the token's K sorted positions inv[n*K+k].  Each lane holds
// 16 elements of a 128-group (8 lanes per group), so every code store is 16 bytes; each lane
// loads UNR groups' slices before any store.
template <typename T, int UNR>
__global__ __launch_bounds__(256) void dispatch_quant_rows_kernel(const T* __restrict__ x, int64_t N, int64_t D,
                                                                  const int32_t* __restrict__ inv, int K,
                                                                  uint8_t* __restrict__ outq,
                                                                  float* __restrict__ outs) {
  constexpr int EPL = 16, LPG = 8, GPW = 8, NLD = EPL * (int)sizeof(T) / 16;  // 16-byte loads per slice
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPG, gl = lane % LPG;
  const int64_t ng = D / 128;
  const int64_t total = N * ng;
  const int64_t M = N * (int64_t)K;
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
      m = max8_lanes(m);
      float sc = m / 448.0f;
      if (sc == 0.0f) sc = 1.0f;
      u32x4 q;
      if (__builtin_expect(div_rn_ok(sc), 1)) {
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
      for (int k = 0; k < K; ++k) {
        const int64_t j = inv[r * K + k];
        if (j < 0 || j >= M) continue;
        *(u32x4*)(outq + j * D + g * 128 + gl * EPL) = q;
        if (gl == 0) outs[j * ng + g] = sc;
      }
    }
  }
}

// out[index[j]] = src[j]
template <typename VT>
__global__ __launch_bounds__(256) void scatter_rows_kernel(
    const char* __restrict__ src, int64_t rows, int64_t row_bytes,
    const int32_t* __restrict__ index, char* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = row_bytes / (int64_t)sizeof(VT);
  const int64_t wave_id = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t j = wave_id; j < rows; j += nwaves) {
    const int64_t d = index[j];
    if (d < 0 || d >= rows) continue;
    const VT* s = (const VT*)(src + j * row_bytes);
    VT* o = (VT*)(out + d * row_bytes);
    for (int64_t c = lane; c < nvec; c += 64) o[c] = s[c];
  }
}

__global__ void invert_perm_kernel(const int32_t* __restrict__ perm, int64_t M, int32_t* __restrict__ inv) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < M) {
    const int64_t p = perm[j];
    if (p >= 0 && p < M) inv[p] = (int32_t)j;
  }
}

static int launch_gather(const void* src, int64_t src_rows, int64_t row_bytes, const int32_t* index,
                         int64_t rows, int64_t div, void* out, hipStream_t st) {
  if (rows == 0 || row_bytes == 0) return MTX_OK;
  const int64_t waves = rows;
  int64_t blocks = ceil_div(waves, 4);
  if (blocks > 65536) blocks = 65536;
  const bool a16 = (row_bytes % 16 == 0) && ((uintptr_t)src % 16 == 0) && ((uintptr_t)out % 16 == 0);
  const bool a4 = (row_bytes % 4 == 0) && ((uintptr_t)src % 4 == 0) && ((uintptr_t)out % 4 == 0);
  if (a16) {
    const int64_t cpr = row_bytes / 16;
    int shift = -1;
    if ((cpr & (cpr - 1)) == 0) {
      shift = 0;
      while ((int64_t(1) << shift) < cpr) ++shift;
    }
    constexpr int UNR = 8;
    int64_t gb = ceil_div(rows * cpr, 256 * UNR);
    if (gb > 16384) gb = 16384;
    hipLaunchKernelGGL(gather_chunks_kernel<UNR>, dim3(gb), dim3(256), 0, st, (const char*)src, src_rows, cpr,
                       shift, index, rows, div, (char*)out);
  } else if (a4)
    hipLaunchKernelGGL(gather_rows_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const char*)src,
                       src_rows, row_bytes, index, rows, div, (char*)out);
  else
    hipLaunchKernelGGL(gather_rows_kernel<uint8_t>, dim3(blocks), dim3(256), 0, st, (const char*)src,
                       src_rows, row_bytes, index, rows, div, (char*)out);
  return check_launch();
}

// ---- unroute -------------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float ldf(const T* p, int64_t i);
template <> __device__ __forceinline__ float ldf<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ldf<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T> __device__ __forceinline__ void stf(T* p, int64_t i, float v);
template <> __device__ __forceinline__ void stf<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void stf<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

// Load 8 consecutive elements as floats (aligned 16B / 32B vector loads).
__device__ __forceinline__ void load8(const float* p, float* o) {
  const float4 a = ((const float4*)p)[0], b = ((const float4*)p)[1];
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void load8(const uint16_t* p, float* o) {
  const uint4 a = *(const uint4*)p;
  const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(u[i] << 16);
    o[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void store8(float* p, const float* v) {
  ((float4*)p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  ((float4*)p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void store8(uint16_t* p, const float* v) {
  *(uint4*)p = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                          pack_bf16x2(v[6], v[7]));
}

// Optional [N, D] addend of the combine (F32 or BF16; p == nullptr: none), added in f32 after
// the k-sum: out = sum_k w*Y + addend, the `routed_out + shared_out` of MoEBlock.__call__
// (bzantium/mintext mintext/modules/moe.py:256-258) in one pass.
struct Addend {
  const void* p;
  int dt;
};
__device__ __forceinline__ void add8(const Addend& a, int64_t off, float* acc) {
  if (!a.p) return;
  float v[8];
  if (a.dt == MTX_BF16) load8((const uint16_t*)a.p + off, v);
  else load8((const float*)a.p + off, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
}
__device__ __forceinline__ float add1(const Addend& a, int64_t i, float acc) {
  return a.p ? acc + load_as_f32(a.p, i, a.dt) : acc;
}

// One wave per token; VEC8 = D % 8 == 0 and aligned pointers.  With KMAX > 0 (K <= KMAX) the
// token's K row indices and weights are read first and the K rows of each 512-element slice are
// loaded together (K independent 16-byte loads in flight per lane) before they are summed in
// k order; the arithmetic is the same fmaf chain as the generic path.
template <typename YT, typename WT, typename OT, bool VEC8, int KMAX>
__global__ __launch_bounds__(256) void unroute_kernel(
    const YT* __restrict__ Y, const int32_t* __restrict__ inv, const WT* __restrict__ w,
    int64_t N, int K, int64_t D, OT* __restrict__ out, Addend add) {
  const int lane = threadIdx.x & 63;
  const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (n >= N) return;
  const int64_t M = N * (int64_t)K;
  if constexpr (VEC8 && KMAX > 0) {
    int64_t jj[KMAX];
    float ww[KMAX];
    bool ok[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      ok[k] = false;
      jj[k] = 0;
      ww[k] = 0.0f;
      if (k < K) {
        const int64_t j = inv[n * K + k];
        ok[k] = (j >= 0 && j < M);
        jj[k] = ok[k] ? j : 0;
        ww[k] = w ? ldf<WT>(w, n * K + k) : 1.0f;
      }
    }
    // S slices of 512 elements per step, so that S*K 16-byte loads are in flight per lane
    constexpr int S = KMAX >= 8 ? 1 : 8 / KMAX;
    for (int64_t d0 = (int64_t)lane * 8; d0 < D; d0 += 512 * S) {
      float y[S][KMAX][8];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int k = 0; k < KMAX; ++k)
          if (k < K && d0 + 512 * s < D) load8(Y + jj[k] * D + d0 + 512 * s, y[s][k]);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int64_t d = d0 + 512 * s;
        if (d >= D) break;
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int k = 0; k < KMAX; ++k)
          if (k < K && ok[k]) {
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = fmaf(ww[k], y[s][k][i], acc[i]);
          }
        add8(add, n * D + d, acc);
        store8(out + n * D + d, acc);
      }
    }
  } else if constexpr (VEC8) {
    for (int64_t d = (int64_t)lane * 8; d < D; d += 512) {
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
      for (int k = 0; k < K; ++k) {
        const int64_t j = inv[n * K + k];
        const float wk = w ? ldf<WT>(w, n * K + k) : 1.0f;
        if (j < 0 || j >= M) continue;
        float y[8];
        load8(Y + j * D + d, y);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(wk, y[i], acc[i]);
      }
      add8(add, n * D + d, acc);
      store8(out + n * D + d, acc);
    }
  } else {
    for (int64_t d = lane; d < D; d += 64) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) {
        const int64_t j = inv[n * K + k];
        const float wk = w ? ldf<WT>(w, n * K + k) : 1.0f;
        if (j < 0 || j >= M) continue;
        acc = fmaf(wk, ldf<YT>(Y, j * D + d), acc);
      }
      stf<OT>(out, n * D + d, add1(add, n * D + d, acc));
    }
  }
}

// Row-wise combine for bf16 expert outputs: SPLIT waves per token, each owning a contiguous
// 1/SPLIT of the row (more waves in flight than one per token: C2 combine 52 -> 49 us with 4,
// C4 114 -> 110 us with 2); the K row pieces of the token are requested whole (S consecutive
// 1 KB slices back to back, kept packed in registers), so each gathered piece reaches HBM as one
// contiguous burst rather than as slices a latency apart.  Then the slices are summed in k
// order with the same fmaf chain as unroute_kernel.  Needs D % (8 * SPLIT) == 0.
template <typename WT, typename OT, int KMAX, int S, int SPLIT>
__global__ __launch_bounds__(256) void unroute_rows_kernel(
    const uint16_t* __restrict__ Y, const int32_t* __restrict__ inv, const WT* __restrict__ w,
    int64_t N, int K, int64_t D, OT* __restrict__ out, Addend add) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n = gw / SPLIT;
  if (n >= N) return;
  const int64_t dbeg = (gw % SPLIT) * (D / SPLIT), dend = dbeg + D / SPLIT;
  const int64_t M = N * (int64_t)K;
  int64_t jj[KMAX];
  float ww[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    jj[k] = -1;
    ww[k] = 0.0f;
    if (k < K) {
      const int64_t j = inv[n * K + k];
      jj[k] = (j >= 0 && j < M) ? j : -1;
      ww[k] = w ? ldf<WT>(w, n * K + k) : 1.0f;
    }
  }
  for (int64_t d0 = dbeg + (int64_t)lane * 8; d0 < dend; d0 += 512 * S) {
    u32x4 q[KMAX][S];
#pragma unroll
    for (int k = 0; k < KMAX; ++k)
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (jj[k] >= 0 && d0 + 512 * s < dend)  // read once: non-temporal (C4 combine 136 -> 113 us)
          q[k][s] = __builtin_nontemporal_load((const u32x4*)(Y + jj[k] * D + d0 + 512 * s));
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int64_t d = d0 + 512 * s;
      if (d >= dend) break;
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int k = 0; k < KMAX; ++k)
        if (jj[k] >= 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[2 * i] = fmaf(ww[k], __uint_as_float(q[k][s][i] << 16), acc[2 * i]);
            acc[2 * i + 1] = fmaf(ww[k], __uint_as_float(q[k][s][i] & 0xffff0000u), acc[2 * i + 1]);
          }
        }
      add8(add, n * D + d, acc);
      // bf16 output (the route VJP's dx, written once): non-temporal (C4 109 -> 102 us, C2 / C3
      // -1 to -3 %); the f32 combine of the forward layer keeps plain stores, which measured
      // faster inside the layer
      if constexpr (std::is_same<OT, uint16_t>::value) st8_nt(out + n * D, d, acc);
      else store8(out + n * D + d, acc);
    }
  }
}

template <typename YT, typename WT, typename OT>
static void launch_unroute_t(const void* Y, const int32_t* inv, const void* w, int64_t N, int K,
                             int64_t D, void* out, Addend add, hipStream_t st) {
  const int64_t blocks = ceil_div(N, 4);
  const bool v8 = (D % 8 == 0) && ((uintptr_t)Y % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                  ((uintptr_t)add.p % 16 == 0);
#define MTX_UNROUTE(V, KM)                                                                                  \
  hipLaunchKernelGGL((unroute_kernel<YT, WT, OT, V, KM>), dim3(blocks), dim3(256), 0, st, (const YT*)Y, inv, \
                     (const WT*)w, N, K, D, (OT*)out, add)
  if (std::is_same<YT, uint16_t>::value && v8 && K <= 8) {
#define MTX_UNROUTE_ROWS_L(KM, SS, SP, WPB)                                                                   \
  hipLaunchKernelGGL((unroute_rows_kernel<WT, OT, KM, SS, SP>), dim3(ceil_div(N * SP, WPB)), dim3(64 * WPB), 0, \
                     st, (const uint16_t*)Y, inv, (const WT*)w, N, K, D, (OT*)out, add)
    // per token: K <= 2, four waves of 2 x 2 KB steps, one wave per workgroup (one wave of
    // 2 x 4 KB: 52 us on C2, of 2 x 8 KB or 2 x 1 KB slower still; eight waves of 1 KB: 51 us;
    // four waves per workgroup: 2 % slower); K <= 8, two waves of 8 x 2 KB (one wave of 8 x 4 KB:
    // C4 114 us, C3 120 us; four waves: 122-126 us)
    if (K <= 2 && D % 32 == 0) MTX_UNROUTE_ROWS_L(2, 2, 4, 1);
    else if (K <= 2) MTX_UNROUTE_ROWS_L(2, 4, 1, 4);
    else if (K <= 4) MTX_UNROUTE_ROWS_L(4, 8, 1, 4);
    else if (D % 16 == 0) MTX_UNROUTE_ROWS_L(8, 2, 2, 4);
    else MTX_UNROUTE_ROWS_L(8, 4, 1, 4);
#undef MTX_UNROUTE_ROWS_L
  } else if (v8 && K <= 2) MTX_UNROUTE(true, 2);
  else if (v8 && K <= 4) MTX_UNROUTE(true, 4);
  else if (v8 && K <= 8) MTX_UNROUTE(true, 8);
  else if (v8) MTX_UNROUTE(true, 0);
  else MTX_UNROUTE(false, 0);
#undef MTX_UNROUTE
}

// unroute backward, one wave per token n (reference VJP of moe_dispatch.py:102-111):
//   dY[inv[n*K+k], :] = w[n,k] * dout[n, :]
//   dw[n,k]          = sum_d dout[n,d] * Y[inv[n*K+k], d]      (f32 math)
template <typename GT, typename YT, typename WT>
__global__ __launch_bounds__(256) void unroute_bwd_kernel(
    const GT* __restrict__ dout, const YT* __restrict__ Y, const int32_t* __restrict__ inv,
    const WT* __restrict__ w, int64_t N, int K, int64_t D, YT* __restrict__ dY, WT* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (n >= N) return;
  const int64_t M = N * (int64_t)K;
  for (int k = 0; k < K; ++k) {
    const int64_t j = inv[n * K + k];
    if (j < 0 || j >= M) continue;
    const float wk = ldf<WT>(w, n * K + k);
    float dot = 0.0f;
    for (int64_t d = lane; d < D; d += 64) {
      const float g = ldf<GT>(dout, n * D + d);
      dot = fmaf(g, ldf<YT>(Y, j * D + d), dot);
      stf<YT>(dY, j * D + d, wk * g);
    }
    if (dw) {
      for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
      if (lane == 0) stf<WT>(dw, n * K + k, dot);
    }
  }
}

// The same VJP for D % 8 == 0, 16-byte aligned rows and K <= KM: each lane moves eight
// consecutive elements per access (16-byte loads and stores) and reads its slice of dout once
// for all K copies of the token, so every byte moves once: N*D of dout, M*D of Y, M*D of dY.
// WPT waves share a token (its 16-byte chunks dealt round-robin), for more loads in flight per
// token; their partial d_w sums are added in wave order through LDS.
template <typename GT, typename YT, typename WT, int KM, int WPT>
__global__ __launch_bounds__(256) void unroute_bwd_vec_kernel(
    const GT* __restrict__ dout, const YT* __restrict__ Y, const int32_t* __restrict__ inv,
    const WT* __restrict__ w, int64_t N, int K, int64_t D, YT* __restrict__ dY, WT* __restrict__ dw) {
  static_assert(WPT == 1 || WPT == 2 || WPT == 4, "waves per token");
  __shared__ float s_dot[4][KM];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave % WPT;
  const int64_t n = (int64_t)blockIdx.x * (4 / WPT) + wave / WPT;
  const bool live = n < N;  // no early return: the waves meet at a barrier below
  const int64_t M = N * (int64_t)K;
  int64_t j[KM];
  float wk[KM], dot[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    j[k] = -1;
    wk[k] = 0.0f;
    dot[k] = 0.0f;
    if (live && k < K) {
      const int64_t jj = inv[n * K + k];
      if (jj >= 0 && jj < M) {  // rows outside [0, M) are skipped, as in the scalar kernel
        j[k] = jj;
        wk[k] = ldf<WT>(w, n * K + k);
      }
    }
  }
  if (live) {
    // two of the lane's chunks per pass (more loads in flight per lane: C4 268 -> 248 us); d_sorted
    // is written once, with non-temporal stores (C2 83 -> 61 us, C4 248 -> 245 us, C3 unchanged);
    // the expert rows are read once, with non-temporal loads when K > 2 (C3 217 -> 196 us, C4 245
    // -> 222 us; C2 +1 %, so plain there; non-temporal dout loads gave nothing).  Every row's loads
    // of a pass are issued before its first store, from rows that are always in bounds (a skipped
    // row reads the token's first kept row, unused), so that 2 KM loads per lane are in flight
    // instead of two per row in turn.
    int64_t jl[KM];
    int64_t j0 = 0;
#pragma unroll
    for (int k = KM - 1; k >= 0; --k) j0 = j[k] >= 0 ? j[k] : j0;
#pragma unroll
    for (int k = 0; k < KM; ++k) jl[k] = j[k] >= 0 ? j[k] : j0;
    const GT* g_row = dout + n * D;
    constexpr int64_t step = 64 * 8 * WPT;
    for (int64_t c = ((int64_t)part * 64 + lane) * 8; c < D; c += 2 * step) {
      const bool two = c + step < D;  // the lane's last pass may hold one chunk
      const int64_t c2 = two ? c + step : c;  // (one chunk: the second loads re-read the first)
      float g[8], g2[8];
      ld8(g_row, c, g);
      ld8(g_row, c2, g2);
      float y[KM][8], y2[KM][8];
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        if constexpr (KM > 2) {
          ld8_nt(Y + jl[k] * D, c, y[k]);
          ld8_nt(Y + jl[k] * D, c2, y2[k]);
        } else {
          ld8(Y + jl[k] * D, c, y[k]);
          ld8(Y + jl[k] * D, c2, y2[k]);
        }
      }
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        float o[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          dot[k] = fmaf(g[q], y[k][q], dot[k]);
          o[q] = wk[k] * g[q];
        }
        if (j[k] >= 0) st8_nt(dY + j[k] * D, c, o);
        if (two) {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            dot[k] = fmaf(g2[q], y2[k][q], dot[k]);
            o[q] = wk[k] * g2[q];
          }
          if (j[k] >= 0) st8_nt(dY + j[k] * D, c2, o);
        }
      }
    }
  }
  if (!dw) return;  // uniform: a kernel argument
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    float s = dot[k];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    dot[k] = s;
  }
  if (WPT > 1) {
    if (lane == 0) {
#pragma unroll
      for (int k = 0; k < KM; ++k) s_dot[wave][k] = dot[k];
    }
    __syncthreads();
    if (part == 0) {
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        float s = s_dot[wave][k];
        for (int p = 1; p < WPT; ++p) s += s_dot[wave + p][k];
        dot[k] = s;
      }
    }
  }
  if (live && part == 0 && lane == 0) {
#pragma unroll
    for (int k = 0; k < KM; ++k)
      if (j[k] >= 0) stf<WT>(dw, n * K + k, dot[k]);
  }
}

// Waves per token of the vector kernel.  Measured on the C2 / C3 / C4 shapes (f32 dout, bf16
// rows): 1 wave 87 / 218 / 293 us, 2 waves 84 / 220 / 262 us, 4 waves 81 / 229 / 265 us.
#ifndef MTX_UB_WPT
#define MTX_UB_WPT 2
#endif
template <typename GT, typename YT, typename WT>
static void launch_unroute_bwd(const void* dout, const void* Y, const int32_t* inv, const void* w, int64_t N, int K,
                               int64_t D, void* dY, void* dw, hipStream_t st) {
  const int64_t blocks = ceil_div(N, 4);
  const bool vec = D % 8 == 0 && K <= 8 && (uintptr_t)dout % 16 == 0 && (uintptr_t)Y % 16 == 0 &&
                   (uintptr_t)dY % 16 == 0;
  constexpr int WPT = MTX_UB_WPT;
#define MTX_UBV(KM)                                                                                             \
  hipLaunchKernelGGL((unroute_bwd_vec_kernel<GT, YT, WT, KM, WPT>), dim3(ceil_div(N, 4 / WPT)), dim3(256), 0, st, \
                     (const GT*)dout, (const YT*)Y, inv, (const WT*)w, N, K, D, (YT*)dY, (WT*)dw)
  if (vec && K <= 2) MTX_UBV(2);
  else if (vec && K <= 4) MTX_UBV(4);
  else if (vec) MTX_UBV(8);
  else
    hipLaunchKernelGGL((unroute_bwd_kernel<GT, YT, WT>), dim3(blocks), dim3(256), 0, st, (const GT*)dout,
                       (const YT*)Y, inv, (const WT*)w, N, K, D, (YT*)dY, (WT*)dw);
#undef MTX_UBV
}

}  // namespace mtx

using namespace mtx;

extern "C" const char* mtx_status_string(int s) {
  switch (s) {
    case MTX_OK: return "ok";
    case MTX_ERR_ARG: return "invalid argument (shape, dtype or combination)";
    case MTX_ERR_WORKSPACE: return "workspace missing or too small";
    case MTX_ERR_UNSUPPORTED: return "unsupported configuration";
    case MTX_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}
extern "C" int mtx_last_hip_error(void) { return g_last_hip_error; }
extern "C" int mtx_version(void) { return 1; }

// ---- streaming copy (HBM ceiling measurement) --------------------------------------------------
// Grid-stride over blocks of 256 x U 16-byte units: each lane issues its U loads, then its U
// stores; NT: non-temporal loads and stores (streamed past the caches).
template <int U, bool NT>
__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                          int64_t n) {
  const int64_t step = (int64_t)gridDim.x * 256 * U;
  for (int64_t b = (int64_t)blockIdx.x * 256 * U + threadIdx.x; b < n; b += step) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = min(b + (int64_t)u * 256, n - 1);  // in bounds; the store below is guarded
      v[u] = NT ? __builtin_nontemporal_load(src + i) : src[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = b + (int64_t)u * 256;
      if (i < n) {
        if (NT) __builtin_nontemporal_store(v[u], dst + i);
        else dst[i] = v[u];
      }
    }
  }
}

extern "C" int mtx_stream_copy(const void* src, void* dst, int64_t nbytes, int variant, int64_t grid, void* stream) {
  if (nbytes < 0 || nbytes % 16 || grid < 0 || grid > 65535 * 16) return MTX_ERR_ARG;
  if (nbytes == 0) return MTX_OK;
  if (!src || !dst || ((uintptr_t)src | (uintptr_t)dst) % 16) return MTX_ERR_ARG;
  int u = (variant >> 4) & 15;
  if (u == 0) u = 8;
  const bool nt = variant & 1;
  if (grid == 0) {
    const int ncu = device_cu_count();
    grid = 4 * (ncu > 0 ? ncu : 256);
  }
  const int64_t n = nbytes / 16;
  hipStream_t st = (hipStream_t)stream;
  const u32x4* s = (const u32x4*)src;
  u32x4* d = (u32x4*)dst;
#define MTX_SC(U)                                                                                          \
  do {                                                                                                     \
    if (nt) hipLaunchKernelGGL((stream_copy_kernel<U, true>), dim3((unsigned)grid), dim3(256), 0, st, s, d, n); \
    else hipLaunchKernelGGL((stream_copy_kernel<U, false>), dim3((unsigned)grid), dim3(256), 0, st, s, d, n); \
  } while (0)
  if (u <= 2) MTX_SC(2);
  else if (u <= 4) MTX_SC(4);
  else if (u <= 8) MTX_SC(8);
  else MTX_SC(16);
#undef MTX_SC
  return check_launch();
}

// Workspace: per-chunk bucket counts, then room for the inverse permutation (used when the
// caller passes inverse == NULL, since the row dispatch runs in token order).
extern "C" int64_t mtx_route_workspace_size(int64_t N, int64_t K, int64_t E) {
  if (N < 0 || K < 1 || E < 1) return -1;
  return route_plan(N, K, E).ws_counts + round_up(N * K * 4, 256);
}

// Stable counting sort of topk_idx: sort_indices, group_sizes and the inverse permutation.
static int route_permutation(const RoutePlan& p, const int32_t* topk_idx, int64_t E, int32_t* counts,
                             int32_t* sort_indices, int32_t* group_sizes, int32_t* inverse, hipStream_t st) {
  // One launch instead of three (count, scan, scatter) while one CU's ballot work (ids x buckets)
  // stays below their fixed cost: about 3 us at 512 ids x 9 buckets and 16 us at 16384 x 9
  // against about 14 us for the three kernels.
  if (E <= 32 && p.M * (E + 1) <= 36864) {
    const size_t shm = (size_t)round_up(p.M > 0 ? p.M : 1, 16);
#define MTX_SMALL(NBT)                                                                                      \
  hipLaunchKernelGGL(route_small_kernel<NBT>, dim3(1), dim3(1024), shm, st, topk_idx, (int)p.M, (int)E, \
                     sort_indices, inverse, group_sizes)
    if (E + 1 <= 9) MTX_SMALL(9);
    else if (E + 1 <= 17) MTX_SMALL(17);
    else MTX_SMALL(33);
#undef MTX_SMALL
    return check_launch();
  }
  const size_t hist_shm = (size_t)p.nb * sizeof(int);
  hipLaunchKernelGGL(route_count_kernel, dim3(p.nchunks), dim3(kRouteThreads), hist_shm, st,
                     topk_idx, p.M, (int)E, p.nb, p.chunk, p.nchunks, p.cstride, counts);
  int nbits = 0;
  while ((1 << nbits) < p.nb) ++nbits;
  const size_t sc_shm = ((size_t)6 * p.nb + 2 * (size_t)p.nb * (p.cstride / 4)) * sizeof(int);
  // M == 0: one chunk with no ids still writes the zero group sizes
  hipLaunchKernelGGL(route_scatter_kernel, dim3(p.nchunks), dim3(kRouteThreads), sc_shm, st, topk_idx,
                     p.M, (int)E, p.nb, nbits, p.chunk, p.cstride, counts, sort_indices, inverse, group_sizes);
  return check_launch();
}

extern "C" int mtx_route(const void* tokens, int dtype, const int32_t* topk_idx,
                         int64_t N, int64_t D, int64_t K, int64_t E,
                         void* sorted_tokens, int32_t* sort_indices, int32_t* group_sizes,
                         int32_t* inverse, const float* token_scales, float* sorted_scales,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  if (N < 0 || D < 0 || K < 1 || E < 1 || E > 1023) return MTX_ERR_ARG;
  if (dtype_size(dtype) == 0) return MTX_ERR_ARG;
  if ((tokens == nullptr) != (sorted_tokens == nullptr)) return MTX_ERR_ARG;
  if ((token_scales == nullptr) != (sorted_scales == nullptr)) return MTX_ERR_ARG;
  if (token_scales && D % 128 != 0) return MTX_ERR_ARG;
  if (N * K > INT32_MAX) return MTX_ERR_ARG;
  // no ids (N == 0): only the E zero group sizes are written; the other buffers may be empty
  if (!group_sizes || (N * K > 0 && (!sort_indices || !topk_idx))) return MTX_ERR_ARG;
  const RoutePlan p = route_plan(N, K, E);
  if (!workspace || workspace_bytes < mtx_route_workspace_size(N, K, E)) return MTX_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  int32_t* counts = (int32_t*)workspace;
  if (!inverse && (tokens || token_scales)) inverse = (int32_t*)((char*)workspace + p.ws_counts);
  int rc = route_permutation(p, topk_idx, E, counts, sort_indices, group_sizes, inverse, st);
  if (rc != MTX_OK) return rc;
  if (p.M == 0 || (!tokens && !token_scales)) return MTX_OK;
  const int64_t row_bytes = D * dtype_size(dtype);
  const bool a16 = (!tokens || ((row_bytes % 16 == 0) && (uintptr_t)tokens % 16 == 0 &&
                                (uintptr_t)sorted_tokens % 16 == 0)) &&
                   (!token_scales || ((D / 128) % 4 == 0 && (uintptr_t)token_scales % 16 == 0 &&
                                      (uintptr_t)sorted_scales % 16 == 0));
  if (!a16) {  // unaligned rows: destination-order gathers
    if (tokens) {
      rc = launch_gather(tokens, N, row_bytes, sort_indices, p.M, K, sorted_tokens, st);
      if (rc != MTX_OK) return rc;
    }
    if (token_scales) {
      rc = launch_gather(token_scales, N, (D / 128) * 4, sort_indices, p.M, K, sorted_scales, st);
      if (rc != MTX_OK) return rc;
    }
    return MTX_OK;
  }
  const int64_t cpr = tokens ? row_bytes / 16 : 0;
  const int64_t spr = token_scales ? (D / 128) * 4 / 16 : 0;
  int shift = -1;
  if (cpr > 0 && (cpr & (cpr - 1)) == 0) {
    shift = 0;
    while ((int64_t(1) << shift) < cpr) ++shift;
  }
  constexpr int UNR = 4;
  int64_t gb = ceil_div(N * (cpr + spr), 256 * UNR);
  if (gb > 16384) gb = 16384;
  if (gb < 1) gb = 1;
  hipLaunchKernelGGL(dispatch_rows_kernel<UNR>, dim3(gb), dim3(256), 0, st, (const u32x4*)tokens, N, cpr, shift,
                     (const u32x4*)token_scales, spr, inverse, (int)K, (u32x4*)sorted_tokens,
                     (u32x4*)sorted_scales);
  return check_launch();
}

extern "C" int mtx_route_quant_fp8(const void* tokens, int dtype, const int32_t* topk_idx, int64_t N,
                                   int64_t D, int64_t K, int64_t E, uint8_t* sorted_q, float* sorted_scales,
                                   int32_t* sort_indices, int32_t* group_sizes, int32_t* inverse,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  if (N < 0 || D < 0 || K < 1 || E < 1 || E > 1023) return MTX_ERR_ARG;
  if (dtype != MTX_F32 && dtype != MTX_BF16) return MTX_ERR_ARG;
  if (D % 128 != 0 || N * K > INT32_MAX) return MTX_ERR_ARG;
  if (!group_sizes || (N > 0 && (!sort_indices || !topk_idx))) return MTX_ERR_ARG;
  if (N > 0 && D > 0 && (!tokens || !sorted_q || !sorted_scales)) return MTX_ERR_ARG;
  if ((uintptr_t)tokens % 16 != 0 || (uintptr_t)sorted_q % 16 != 0 || (uintptr_t)sorted_scales % 4 != 0)
    return MTX_ERR_ARG;
  const RoutePlan p = route_plan(N, K, E);
  if (!workspace || workspace_bytes < mtx_route_workspace_size(N, K, E)) return MTX_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  int32_t* counts = (int32_t*)workspace;
  if (!inverse) inverse = (int32_t*)((char*)workspace + p.ws_counts);
  int rc = route_permutation(p, topk_idx, E, counts, sort_indices, group_sizes, inverse, st);
  if (rc != MTX_OK) return rc;
  if (p.M == 0 || D == 0) return MTX_OK;
  constexpr int UNR = 4;
  const int64_t groups = N * (D / 128);
  int64_t gb = ceil_div(groups, (int64_t)8 * 4 * UNR);  // 8 groups per wave and step, 4 waves
  if (gb > 16384) gb = 16384;
  if (dtype == MTX_BF16)
    hipLaunchKernelGGL((dispatch_quant_rows_kernel<uint16_t, UNR>), dim3(gb), dim3(256), 0, st,
                       (const uint16_t*)tokens, N, D, inverse, (int)K, sorted_q, sorted_scales);
  else
    hipLaunchKernelGGL((dispatch_quant_rows_kernel<float, UNR>), dim3(gb), dim3(256), 0, st, (const float*)tokens,
                       N, D, inverse, (int)K, sorted_q, sorted_scales);
  return check_launch();
}

extern "C" int mtx_gather_rows(const void* src, int dtype, int64_t src_rows, int64_t D,
                               const int32_t* index, int64_t rows, int64_t div, void* out, void* stream) {
  if (src_rows < 0 || D < 0 || rows < 0 || div < 1 || dtype_size(dtype) == 0) return MTX_ERR_ARG;
  if (rows > 0 && (!src || !index || !out)) return MTX_ERR_ARG;
  return launch_gather(src, src_rows, D * dtype_size(dtype), index, rows, div, out, (hipStream_t)stream);
}

extern "C" int mtx_scatter_rows(const void* src, int dtype, int64_t rows, int64_t D,
                                const int32_t* index, void* out, void* stream) {
  if (rows < 0 || D < 0 || dtype_size(dtype) == 0) return MTX_ERR_ARG;
  if (rows == 0 || D == 0) return MTX_OK;
  if (!src || !index || !out) return MTX_ERR_ARG;
  const int64_t rb = D * dtype_size(dtype);
  int64_t blocks = ceil_div(rows, 4);
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  const bool a16 = (rb % 16 == 0) && ((uintptr_t)src % 16 == 0) && ((uintptr_t)out % 16 == 0);
  const bool a4 = (rb % 4 == 0) && ((uintptr_t)src % 4 == 0) && ((uintptr_t)out % 4 == 0);
  if (a16)
    hipLaunchKernelGGL(scatter_rows_kernel<u32x4>, dim3(blocks), dim3(256), 0, st, (const char*)src, rows, rb,
                       index, (char*)out);
  else if (a4)
    hipLaunchKernelGGL(scatter_rows_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const char*)src, rows,
                       rb, index, (char*)out);
  else
    hipLaunchKernelGGL(scatter_rows_kernel<uint8_t>, dim3(blocks), dim3(256), 0, st, (const char*)src, rows,
                       rb, index, (char*)out);
  return check_launch();
}

extern "C" int mtx_invert_permutation(const int32_t* perm, int64_t M, int32_t* inverse, void* stream) {
  if (M < 0 || M > INT32_MAX) return MTX_ERR_ARG;
  if (M == 0) return MTX_OK;
  if (!perm || !inverse) return MTX_ERR_ARG;
  hipLaunchKernelGGL(invert_perm_kernel, dim3(ceil_div(M, 256)), dim3(256), 0, (hipStream_t)stream, perm, M,
                     inverse);
  return check_launch();
}

static int unroute_entry(const void* sorted_output, int y_dtype, const int32_t* inverse, const void* topk_w,
                         int w_dtype, int64_t N, int64_t K, int64_t D, Addend add, void* out, int out_dtype,
                         void* stream) {
  if (N < 0 || K < 1 || K > 1024 || D < 0) return MTX_ERR_ARG;
  if ((y_dtype != MTX_F32 && y_dtype != MTX_BF16) || (w_dtype != MTX_F32 && w_dtype != MTX_BF16) ||
      (out_dtype != MTX_F32 && out_dtype != MTX_BF16) || (add.p && add.dt != MTX_F32 && add.dt != MTX_BF16))
    return MTX_ERR_ARG;
  if (N == 0 || D == 0) return MTX_OK;
  if (!sorted_output || !inverse || !out) return MTX_ERR_ARG;  // topk_w == NULL: unit weights
  hipStream_t st = (hipStream_t)stream;
  const int k = (int)K;
#define MTX_UNR(YT, WT, OT) launch_unroute_t<YT, WT, OT>(sorted_output, inverse, topk_w, N, k, D, out, add, st)
  if (y_dtype == MTX_BF16) {
    if (w_dtype == MTX_F32) { if (out_dtype == MTX_F32) MTX_UNR(uint16_t, float, float); else MTX_UNR(uint16_t, float, uint16_t); }
    else { if (out_dtype == MTX_F32) MTX_UNR(uint16_t, uint16_t, float); else MTX_UNR(uint16_t, uint16_t, uint16_t); }
  } else {
    if (w_dtype == MTX_F32) { if (out_dtype == MTX_F32) MTX_UNR(float, float, float); else MTX_UNR(float, float, uint16_t); }
    else { if (out_dtype == MTX_F32) MTX_UNR(float, uint16_t, float); else MTX_UNR(float, uint16_t, uint16_t); }
  }
#undef MTX_UNR
  return check_launch();
}

extern "C" int mtx_unroute(const void* sorted_output, int y_dtype, const int32_t* inverse,
                           const void* topk_w, int w_dtype, int64_t N, int64_t K, int64_t D,
                           void* out, int out_dtype, void* stream) {
  return unroute_entry(sorted_output, y_dtype, inverse, topk_w, w_dtype, N, K, D, Addend{nullptr, 0}, out,
                       out_dtype, stream);
}

extern "C" int mtx_unroute_add(const void* sorted_output, int y_dtype, const int32_t* inverse,
                               const void* topk_w, int w_dtype, int64_t N, int64_t K, int64_t D,
                               const void* addend, int add_dtype, void* out, int out_dtype, void* stream) {
  if (!addend) return MTX_ERR_ARG;
  return unroute_entry(sorted_output, y_dtype, inverse, topk_w, w_dtype, N, K, D, Addend{addend, add_dtype}, out,
                       out_dtype, stream);
}

extern "C" int mtx_unroute_bwd(const void* dout, int g_dtype, const void* sorted_output, int y_dtype,
                               const int32_t* inverse, const void* topk_w, int w_dtype, int64_t N, int64_t K,
                               int64_t D, void* d_sorted, void* d_w, void* stream) {
  if (N < 0 || K < 1 || D < 0) return MTX_ERR_ARG;
  if ((g_dtype != MTX_F32 && g_dtype != MTX_BF16) || (y_dtype != MTX_F32 && y_dtype != MTX_BF16) ||
      (w_dtype != MTX_F32 && w_dtype != MTX_BF16))
    return MTX_ERR_ARG;
  if (N == 0) return MTX_OK;
  if (!dout || !sorted_output || !inverse || !topk_w || !d_sorted) return MTX_ERR_ARG;
  if (K > INT32_MAX) return MTX_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int k = (int)K;
#define MTX_UB(GT, YT, WT) launch_unroute_bwd<GT, YT, WT>(dout, sorted_output, inverse, topk_w, N, k, D, d_sorted, d_w, st)
  if (g_dtype == MTX_F32) {
    if (y_dtype == MTX_F32) { if (w_dtype == MTX_F32) MTX_UB(float, float, float); else MTX_UB(float, float, uint16_t); }
    else { if (w_dtype == MTX_F32) MTX_UB(float, uint16_t, float); else MTX_UB(float, uint16_t, uint16_t); }
  } else {
    if (y_dtype == MTX_F32) { if (w_dtype == MTX_F32) MTX_UB(uint16_t, float, float); else MTX_UB(uint16_t, float, uint16_t); }
    else { if (w_dtype == MTX_F32) MTX_UB(uint16_t, uint16_t, float); else MTX_UB(uint16_t, uint16_t, uint16_t); }
  }
#undef MTX_UB
  return check_launch();
}
