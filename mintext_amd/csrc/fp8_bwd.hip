// Backward of the blockwise-fp8 grouped GEMM on gfx950 (no reference counterpart: the bf16 forms
// are dlhs and tgmm of bzantium/mintext mintext/kernels/grouped_matmul.py:151-187 and :197-235;
// the fp8 conventions are those of the forward, DeepSeek-V3 style blockwise e4m3fn with f32
// scale = amax / 448).
//
// dlhs  dX = dY @ W^T: dY is quantised in 1x128 groups along its row (the reduction), and W in
//       128x128 blocks exactly as for the forward but with its codes kept in W's own layout
//       [E, Kin, Kout] (k-contiguous for this product) and the block-scale grid transposed; the
//       product is then the forward fp8 grouped GEMM (mtx_gmm_fp8) on these operands.
// tgmm  dW[e] = X_e^T @ G_e reduces over the rows of expert e.  Both operands are quantised in
//       groups of 128 consecutive rows of the expert (expert-aligned chunks: chunk j of expert e
//       covers its rows 128j .. 128j+127, the last chunk zero-padded) and transposed per expert so
//       that the reduction is contiguous: expert e's block XT_e [F, 128*n_e] (n_e chunks) starts
//       at byte 128*F*cb[e] (cb[e] = chunks of the experts before e), with one scale per feature
//       and chunk ([F, n_e] at float cb[e]*F; 1x128 along the transposed row), and GT_e [N, 128*n_e]
//       likewise with one scale per 128 features and chunk ([N/128, n_e] at float cb[e]*N/128;
//       128x128 blocks).  Expert-major blocks keep each tile's 256 rows within a few hundred KB
//       (a row-major [F, 128*C] layout put them 128*C bytes apart, one page per row).  The GEMM is
//       the forward kernel's tile loop with a per-expert k-range.
// Both have a power-of-two mode (the "_p2" entry points): every scale is p2_scale(amax) instead of
// amax / 448, and the GEMMs give the scales' exponents to the MFMA's E8M0 operands, as the forward's
// power-of-two mode does (accumulators in true units over the whole reduction).
#include "common.h"
#include "lds_dma.h"
#include "fp8_tile.h"

namespace mtx {
namespace f8b {

typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;


// ---- weights in their own layout ---------------------------------------------------------------
// The 128x128 block (Kin block y, Kout block x) of expert z: the scale of quant_weights_kernel
// (amax / 448 of the same block) and the same codes, written in W's layout [E, Kin, Kout] with the
// scale at [E, Kin/128, Kout/128].
template <typename T, bool P2 = false>
__global__ __launch_bounds__(256) void quant_weights_t_kernel(const T* __restrict__ w, int64_t Kin, int64_t Kout,
                                                              uint8_t* __restrict__ wq, float* __restrict__ ws) {
  __shared__ float red[4];
  using S = q8::TileShape<T>;
  const int64_t e = blockIdx.z, k0 = (int64_t)blockIdx.y * 128, n0 = (int64_t)blockIdx.x * 128;
  const int64_t base = (e * Kin + k0) * Kout + n0;
  q8::Tile<T> t;
  t.load(w + base, Kout, 128);
  float m[S::VE];
  t.col_amax(m);
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < S::VE; ++j) a = fmaxf(a, m[j]);
  const float s = q8::block_scale<P2>(a, red);
  q8::codes_to_global(t, s, wq + base, Kout);
  if (threadIdx.x == 0) ws[(e * (Kin / 128) + blockIdx.y) * (Kout / 128) + blockIdx.x] = s;
}

// ---- expert chunks -----------------------------------------------------------------------------
// One workgroup, E <= 1024: row offsets off[E+1] of the groups (clamped to M like the forward's
// tile builder), chunk bases cb[E+1] (cb[e] = sum of ceil(rows/128) over the experts before e)
// and the experts in descending size order (ties: lower id first), so the longest reductions
// start first; misc[0] = the experts with rows (a prefix of that order), misc[8..15] = 0 (the
// persistent tgmm's tile tickets).
__global__ __launch_bounds__(1024) void chunk_prologue_kernel(const int32_t* __restrict__ gs, int E, int M,
                                                              int* __restrict__ cb, int* __restrict__ off,
                                                              int* __restrict__ order, int* __restrict__ misc) {
  __shared__ long long wsum64[16];
  __shared__ int wsum[16];
  __shared__ int s_rows[1024];
  const int e = threadIdx.x, lane = e & 63, w = e >> 6;
  const int g = (e < E) ? min(max(gs[e], 0), M) : 0;
  long long incl64 = g;
  for (int o = 1; o < 64; o <<= 1) {
    const long long v = __shfl_up(incl64, o);
    if (lane >= o) incl64 += v;
  }
  if (lane == 63) wsum64[w] = incl64;
  __syncthreads();
  if (e == 0) {
    long long run = 0;
    for (int i = 0; i < 16; ++i) { const long long v = wsum64[i]; wsum64[i] = run; run += v; }
  }
  __syncthreads();
  const long long start = incl64 - g + wsum64[w];
  const int r0 = (int)min(start, (long long)M), r1 = (int)min(start + g, (long long)M);
  const int rows = r1 - r0, nch = (rows + 127) / 128;
  s_rows[e] = (e < E) ? rows : -1;
  int incl = nch;
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  if (e == 0) {
    int run = 0;
    for (int i = 0; i < 16; ++i) { const int v = wsum[i]; wsum[i] = run; run += v; }
  }
  __syncthreads();
  if (e < E) {
    cb[e] = incl - nch + wsum[w];
    off[e] = r0;
    if (e == E - 1) {
      cb[E] = incl + wsum[w];
      off[E] = r1;
    }
    int rank = 0;
    for (int h = 0; h < E; ++h) rank += (s_rows[h] > rows || (s_rows[h] == rows && h < e)) ? 1 : 0;
    order[rank] = e;
  }
  const int nrows = __syncthreads_count(e < E && nch >= 1);
  if (e == 0) misc[0] = nrows;
  if (e >= 8 && e < 16) misc[e] = 0;
}

// expert owning chunk c: the last e with cb[e] <= c (experts without chunks share their
// successor's base)
__device__ __forceinline__ int chunk_expert(const int* __restrict__ cb, int E, int c) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cb[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// ---- grouped transposing quantiser -------------------------------------------------------------
// Workgroup (chunk c, 128-feature block fb): chunk j = c - cb[e] of expert e, its rows off[e] + 128j
// .. +127 (rows past the expert are zero) x features fb*128 .. +127 of x [M, F] -> codes at
// xt[128*F*cb[e] + f*128*n_e + 128j + r] (n_e = chunks of expert e).  ROW: scale per feature =
// amax over the chunk's rows / 448 at xts[F*cb[e] + f*n_e + j]; BLOCK: one scale per 128x128 block
// at xts[(F/128)*cb[e] + fb*n_e + j].  Codes are e4m3 of v / scale, scale 1 when the amax is 0.
template <typename T, bool BLOCK, bool P2 = false>
__global__ __launch_bounds__(256) void quant_grouped_t_kernel(const T* __restrict__ x, int F, const int* __restrict__ cb,
                                                              const int* __restrict__ off, int E,
                                                              uint8_t* __restrict__ xt, float* __restrict__ xts) {
  using S = q8::TileShape<T>;
  __shared__ __attribute__((aligned(16))) uint8_t tt[128 * q8::TSTRIDE];
  __shared__ float red[S::TR][128];
  __shared__ float scs[128];
  const int c = blockIdx.x, fb = blockIdx.y, tid = threadIdx.x;
  if (c >= cb[E]) return;  // beyond the chunks of this call's groups
  const int e = chunk_expert(cb, E, c);
  const int j = c - cb[e], ne = cb[e + 1] - cb[e];
  const int rs = off[e] + 128 * j;
  const int nr = min(128, off[e + 1] - rs);
  const int64_t f0 = (int64_t)fb * 128;
  q8::Tile<T> t;
  t.load(x + (int64_t)rs * F + f0, F, nr);
  float m[S::VE];
  t.col_amax(m);
  if (BLOCK) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < S::VE; ++i) a = fmaxf(a, m[i]);
    const float s = q8::block_scale<P2>(a, &red[0][0]);
    q8::codes_to_lds_t(t, [&](int) { return s; }, tt);
    if (tid == 0) xts[(int64_t)(F / 128) * cb[e] + (int64_t)fb * ne + j] = s;
  } else {
#pragma unroll
    for (int i = 0; i < S::VE; ++i) red[t.rl][t.cl * S::VE + i] = m[i];
    __syncthreads();
    if (tid < 128) {
      float a = 0.0f;
#pragma unroll
      for (int r = 0; r < S::TR; ++r) a = fmaxf(a, red[r][tid]);
      const float s = q8::scale_of<P2>(a);
      scs[tid] = s;
      xts[(int64_t)F * cb[e] + (f0 + tid) * ne + j] = s;
    }
    __syncthreads();
    q8::codes_to_lds_t(t, [&](int i) { return scs[t.cl * S::VE + i]; }, tt);
  }
  __syncthreads();
  const int64_t lde = (int64_t)128 * ne;
  q8::lds_t_to_global(tt, xt + (int64_t)128 * F * cb[e] + (int64_t)128 * j + f0 * lde, lde);
}

// ---- tgmm: dW[e] = XT_e GT_e^T over the expert's chunks ---------------------------------------------
// 256x256 output tiles of dW[e] [F, N], 8 waves (2 x 4, 128x64 wave tiles of 32x32 blocks), 64-k
// stages of 256 XT rows and 256 GT rows (32 KB) loaded with global_load_lds_dwordx4 into a 4-deep
// LDS ring three stages ahead; one v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales) per block and
// stage, operands swapped so that each lane owns four consecutive output columns.  The scales of
// chunk j travel with its even stage 2j (global_load_lds_dword: waves 0-3 the 256 XT-row scales,
// wave 4 the two GT-block scales, waves 5-7 a filler load so that every wave issues the same
// number of loads), so no wait on memory is added for them.  Per chunk the accumulators are kept
// in units of the chunk's scale product and moved to the next chunk's units by
// (sa_c / sa_n) * (sb_c / sb_n) (no product of two small scales is formed), the last chunk's
// scales applied at the end.  An expert without rows gives a zero tile.
constexpr int TBM = 256, TBN = 256, TBK = 64, TNST = 4, TPD = 3;
constexpr int TA_BYTES = TBM * TBK, TS_OFF = 2 * TA_BYTES, TSTAGE = TS_OFF + 2048;
__device__ __forceinline__ int t_off(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

struct TArgs {
  const uint8_t* xt;  // expert-major blocks [F, 128 n_e]
  const float* xts;   // expert-major [F, n_e]
  const uint8_t* gt;  // expert-major blocks [N, 128 n_e]
  const float* gts;   // expert-major [N/128, n_e]
  uint16_t* dw;       // [E, F, N] bf16
  const int* cb;      // [E+1]
  const int* order;   // [E]
  int E, F, N;
  int xa, xb;         // XCD rectangles: 0 = row-major tiles, else an xa x xb grid of the tile grid
};

template <bool P2 = false>
__global__ __launch_bounds__(512, 2) void tgmm_fp8_kernel(TArgs p) {
  constexpr int WN = 4, WTM = 128, WTN = 64, TM = 4, TN = 2, LPS = 4;  // data loads per wave and stage
  __shared__ __attribute__((aligned(1024))) char lds[TNST * TSTAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int nf = p.F / TBM, nn = p.N / TBN, per_e = nf * nn;
  const int total = p.E * per_e;
  // consecutive workgroups (which the dispatcher places on consecutive XCDs, x = lid % 8) take
  // consecutive tiles, so the tiles of the large experts, which come first, spread over all XCDs.
  // With xa > 0 (per_e a multiple of 8) XCD x takes the tiles of one (nf/xa) x (nn/xb) rectangle
  // of the expert's tile grid, so that it reads few XT and GT blocks of the expert into its L2.
  const int lid = blockIdx.x;
  if (lid >= total) return;
  const int e = p.order[lid / per_e];
  const int rem = lid % per_e;
  int fb, nb;
  if (p.xa > 0) {
    const int x = rem & 7, q = rem >> 3, rh = nf / p.xa, rw = nn / p.xb;
    fb = (x % p.xa) * rh + q / rw;
    nb = (x / p.xa) * rw + q % rw;
  } else {
    fb = rem / nn;
    nb = rem % nn;
  }
  const int c0 = p.cb[e], nch = p.cb[e + 1] - c0;
  uint16_t* out = p.dw + (int64_t)e * p.F * p.N + (int64_t)fb * TBM * p.N + nb * TBN;
  if (nch <= 0) {  // empty group: dW[e] tile = 0
    for (int i = tid; i < TBM * TBN / 8; i += 512) {
      const int r = i / (TBN / 8), cc = (i % (TBN / 8)) * 8;
      *(u32x4*)(out + (int64_t)r * p.N + cc) = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const int nk = 2 * nch;  // 64-byte stages
  const uint32_t lde = (uint32_t)nch * 128u;  // bytes per row of this expert's blocks
  const uint8_t* xe = p.xt + (int64_t)128 * p.F * c0;
  const uint8_t* ge = p.gt + (int64_t)128 * p.N * c0;

  // per-lane sources: lane l of segment s fills tile row 16s + l/4, chunk slot l%4
  uint32_t aoff[2], boff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int seg = wave * 2 + i;
    const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
    aoff[i] = (uint32_t)(fb * TBM + r) * lde + (uint32_t)(c * 16);
    boff[i] = (uint32_t)(nb * TBN + r) * lde + (uint32_t)(c * 16);
  }
  // this lane's scale source for chunk 0 (one float per chunk after it): waves 0-3 XT row
  // fb*256 + 64*wave + lane, wave 4 the GT block nb*2 + (lane & 1), the others a filler
  const float* sp;
  if (wave < 4) sp = p.xts + (int64_t)p.F * c0 + (int64_t)(fb * TBM + 64 * wave + lane) * nch;
  else if (wave == 4) sp = p.gts + (int64_t)(p.N / 128) * c0 + (int64_t)(nb * 2 + (lane & 1)) * nch;
  else sp = p.xts + (int64_t)p.F * c0;
  const uint32_t lds_base = lds_addr(lds);
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  // stages past the end re-read the last one (in bounds) into a slot that is no longer read;
  // even stages also carry their chunk's scales (LPS + 1 loads per wave)
  auto issue_stage = [&](int kt) {
    const uint32_t st = lds_base + (uint32_t)((kt & (TNST - 1)) * TSTAGE);
    const int k = min(kt, nk - 1);
    const uint32_t kofs = (uint32_t)k * TBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) gload_lds16(xe + aoff[i] + kofs, st + (wave_u * 2 + i) * 1024u);
#pragma unroll
    for (int i = 0; i < 2; ++i) gload_lds16(ge + boff[i] + kofs, st + (uint32_t)TA_BYTES + (wave_u * 2 + i) * 1024u);
    if ((kt & 1) == 0) gload_lds4(sp + (k >> 1), st + (uint32_t)TS_OFF + wave_u * 256u);
  };
  const int frow = lane & 31, fhalf = lane >> 5;
  auto ld32 = [&](const char* base, int r) -> i32x8 {
    const u32x4 lo = *(const u32x4*)(base + t_off(r, 2 * fhalf));
    const u32x4 hi = *(const u32x4*)(base + t_off(r, 2 * fhalf + 1));
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  // rotating fragments: one A set and two B sets; A of row block i is reloaded from the next stage
  // right after its last MFMA, the next stage's B fragments go to the other set, so that the live
  // fragments fit beside the 128 accumulators without serialising every LDS read before its MFMA
  i32x8 fr_a[TM], fr_b[2][TN];
  auto rd_a = [&](int kt, int i) -> i32x8 { return ld32(lds + (kt & (TNST - 1)) * TSTAGE, wm * WTM + i * 32 + frow); };
  auto rd_b = [&](int kt, int j) -> i32x8 {
    return ld32(lds + (kt & (TNST - 1)) * TSTAGE + TA_BYTES, wn * WTN + j * 32 + frow);
  };
  // scales of the chunk whose even stage is kt: this lane's four XT rows and this wave's GT block
  float sa_c[TM], sa_n[TM], sb_c, sb_n;
  auto read_scales = [&](int kt, float* sa, float& sb) {
    const float* sc = (const float*)(lds + (kt & (TNST - 1)) * TSTAGE + TS_OFF);
#pragma unroll
    for (int i = 0; i < TM; ++i) sa[i] = sc[wm * WTM + i * 32 + frow];
    sb = sc[256 + (wn >> 1)];
  };
  // P2: the same scales as E8M0 codes for the MFMA's scale operands -- the lane's four XT-row codes
  // packed one per byte (opsel i) and the wave's GT-block code
  uint32_t ea_c = 0, ea_n = 0, eb_c = 0, eb_n = 0;
  auto read_codes = [&](int kt, uint32_t& ea, uint32_t& eb) {
    const float* sc = (const float*)(lds + (kt & (TNST - 1)) * TSTAGE + TS_OFF);
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) s |= e8m0_of(sc[wm * WTM + i * 32 + frow]) << (8 * i);
    ea = s;
    eb = e8m0_of(sc[256 + (wn >> 1)]);
  };
  // acc += GT_j XT_i scaled by the current chunk's codes (opsel is a constant: one case per i)
  auto mfma_p2 = [&](const i32x8& b, const i32x8& a, const f32x16& c, int i) -> f32x16 {
    switch (i) {
      case 0: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 0, (int)ea_c);
      case 1: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 1, (int)ea_c);
      case 2: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 2, (int)ea_c);
      default: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 3, (int)ea_c);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // One stage: MFMAs of stage kt on fr_a / fr_b[cb] with the fragments of stage kt+1 read in
  // between; at a chunk boundary each accumulator is moved to the new chunk's units one slot ahead
  // of its MFMA, while the previous MFMA runs.
  auto rot_stage = [&](int kt, int cb, bool rescale, const float (&f)[TM]) {
#pragma unroll
    for (int j = 0; j < TN; ++j) fr_b[cb ^ 1][j] = rd_b(kt + 1, j);
    auto rescale_acc = [&](int q) {
      const int i = q / TN, j = q % TN;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] *= f[i];
    };
    if (rescale) rescale_acc(0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (P2)
          acc[i][j] = mfma_p2(fr_b[cb][j], fr_a[i], acc[i][j], i);
        else
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr_b[cb][j], fr_a[i], acc[i][j], 0, 0, 0, 127, 0,
                                                                      127);
        if (rescale && i * TN + j + 1 < TM * TN) rescale_acc(i * TN + j + 1);
      }
      fr_a[i] = rd_a(kt + 1, i);
    }
  };

  // prologue: stages 0 (+ scales), 1, 2 (+ scales); 0 and 1 landed (2's LPS + 1 loads may fly)
#pragma unroll
  for (int s = 0; s < TPD; ++s) issue_stage(s);  // nk >= 2: stages past the end re-read the last
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS + 1));
  __syncthreads();
  if constexpr (P2) read_codes(0, ea_c, eb_c);
  else read_scales(0, sa_c, sb_c);
#pragma unroll
  for (int i = 0; i < TM; ++i) fr_a[i] = rd_a(0, i);
#pragma unroll
  for (int j = 0; j < TN; ++j) fr_b[0][j] = rd_b(0, j);
  for (int kb = 0; kb < nch; ++kb) {
    const int kt = 2 * kb;
    issue_stage(kt + TPD);  // odd stage: LPS loads
    float f[TM];
    if (P2 && kb > 0) {  // true units throughout: only the codes change
      ea_c = ea_n;
      eb_c = eb_n;
      rot_stage(kt, 0, false, f);
    } else if (kb > 0) {
      // (sa_c / sa_n) * (sb_c / sb_n): no product of two small scales is formed
      const float rb = sb_c * __builtin_amdgcn_rcpf(sb_n);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        f[i] = (sa_c[i] * __builtin_amdgcn_rcpf(sa_n[i])) * rb;
        sa_c[i] = sa_n[i];
      }
      sb_c = sb_n;
      rot_stage(kt, 0, true, f);
    } else {
      rot_stage(kt, 0, false, f);
    }
    // stage kt+2 (LPS + 1 loads, issued before stage kt+3) landed; kt+3 may still be in flight.
    // Bare s_barrier: this wave's outstanding LDS reads are the next stage's fragments (visible
    // since the previous barrier) and need not complete before it; a slot is refilled only after
    // every wave's MFMAs consumed the fragments read from it.
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS));
    __builtin_amdgcn_s_barrier();
    issue_stage(kt + 1 + TPD);  // even stage: LPS + 1 loads
    if constexpr (P2) read_codes(kt + 2, ea_n, eb_n);  // the next chunk's codes (past the last: unused)
    else read_scales(kt + 2, sa_n, sb_n);  // the next chunk's scales (past the last: an unused slot)
    rot_stage(kt + 1, 1, false, f);  // its fragment reads of stage kt+2 past the end are unused
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS + 1));  // stage kt+3 landed; kt+4 may still be in flight
    __builtin_amdgcn_s_barrier();
  }
  // every ring load (the ones past the end included) has landed before the ring is reused
  __builtin_amdgcn_s_waitcnt(MTX_VMCNT(0));
  __syncthreads();

  // epilogue: acc[i][j][4g+q] of lane l is dW[row i*32 + l%32][col j*32 + 8g + 4(l/32) + q]; staged
  // through the ring (32 rows x 64 bf16 columns per wave at a time, 16-byte chunk c of row r at
  // chunk c ^ (r & 7)) so that each store writes whole 128-byte row segments
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = P2 ? acc[i][j][v] : (acc[i][j][v] * sa_c[i]) * sb_c;
  char* wst = lds + wave * 4096;
  const uint32_t lo = (uint32_t)(wm * WTM + (lane >> 3)) * (uint32_t)p.N + (uint32_t)(wn * WTN + (lane & 7) * 8);
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
      *(u32x4*)(out + lo + (uint32_t)(i * 32 + rr * 8) * (uint32_t)p.N) = v;
    }
    __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);  // reads done before the next block overwrites
  }
}

// ---- persistent tgmm ---------------------------------------------------------------------------
// The tiles and arithmetic of tgmm_fp8_kernel (the same MFMA sequence per output element, so the
// same bits) with one workgroup per CU and the ring of gmm_fp8_v4_kernel running across tiles: the
// next tile's first three stages are loaded during the current tile's last three, so a tile starts
// without the ring prologue (5.4 us of a C5 tile's 27 us in the per-tile kernel, with 1-2 us
// between workgroups).  The tiles of the experts with rows (misc[0] of them, a prefix of `order`)
// come in tgmm_fp8_kernel's order: XCD x takes tiles 8j + x (the per-tile kernel's XCD of the same
// tile, so the XCD rectangles stay), its workgroups their first j statically and the rest from the
// XCD's ticket counter misc[8 + x], drawn by wave 0 at the start of each epilogue.  An expert
// of one chunk (two stages) is too short for the three-stage lookahead to stay within the next
// tile: around its tiles the ring restarts.  The zero tiles of the experts without rows are
// written first.  misc is written by chunk_prologue_kernel.
template <bool P2 = false>
__global__ __launch_bounds__(512, 2) void tgmm_fp8_p_kernel(TArgs p, int* misc) {
  constexpr int WN = 4, WTM = 128, WTN = 64, TM = 4, TN = 2, LPS = 4;  // data loads per wave and stage
  __shared__ __attribute__((aligned(1024))) char lds[TNST * TSTAGE];
  __shared__ int s_ticket;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const int wm = wave / WN, wn = wave % WN;
  const int nf = p.F / TBM, nn = p.N / TBN, per_e = nf * nn;
  typedef const __attribute__((address_space(4))) int cint_t;
  const int n_rows = __builtin_amdgcn_readfirstlane(*(const cint_t*)(uintptr_t)misc);
  const int total = n_rows * per_e, all = p.E * per_e;
  const int nx = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), q = (int)(blockIdx.x >> 3);

  struct Tile {
    int e, fb, nb, c0, nch;
  };
  // tile lid of tgmm_fp8_kernel's order (experts by descending size, xa x xb XCD rectangles); the
  // read-only lists go through the scalar cache
  auto decode = [&](int lid) -> Tile {
    Tile T;
    const int ei = lid / per_e, rem = lid - ei * per_e;
    T.e = __builtin_amdgcn_readfirstlane(((const cint_t*)(uintptr_t)p.order)[ei]);
    if (p.xa > 0) {
      const int x = rem & 7, qq = rem >> 3, rh = nf / p.xa, rw = nn / p.xb;
      T.fb = (x % p.xa) * rh + qq / rw;
      T.nb = (x / p.xa) * rw + qq % rw;
    } else {
      T.fb = rem / nn;
      T.nb = rem % nn;
    }
    const cint_t* cbp = (const cint_t*)(uintptr_t)p.cb;
    T.c0 = __builtin_amdgcn_readfirstlane(cbp[T.e]);
    T.nch = __builtin_amdgcn_readfirstlane(cbp[T.e + 1]) - T.c0;
    return T;
  };
  struct Src {
    uint32_t aoff[2], boff[2];
    const uint8_t* A;
    const uint8_t* B;
    const float* sb;  // this wave's scale base (uniform) ...
    uint32_t so;      // ... + this lane's byte offset: its scale for chunk 0 (one float per chunk after it)
  };
  // per-lane sources: lane l of segment s fills tile row 16s + l/4, chunk slot l%4; waves 0-3 load
  // the XT-row scales of rows 64w + l, wave 4 the two GT-block scales, the others a filler
  auto make_src = [&](const Tile& T) -> Src {
    Src S;
    const uint32_t lde = (uint32_t)T.nch * 128u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int seg = wave * 2 + i;
      const int r = seg * 16 + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
      S.aoff[i] = (uint32_t)(T.fb * TBM + r) * lde + (uint32_t)(c * 16);
      S.boff[i] = (uint32_t)(T.nb * TBN + r) * lde + (uint32_t)(c * 16);
    }
    S.A = p.xt + (int64_t)128 * p.F * T.c0;
    S.B = p.gt + (int64_t)128 * p.N * T.c0;
    if (wave_u < 4) {
      S.sb = p.xts + (int64_t)p.F * T.c0;
      S.so = (uint32_t)(T.fb * TBM + 64 * wave + lane) * (uint32_t)T.nch * 4u;
    } else if (wave_u == 4) {
      S.sb = p.gts + (int64_t)(p.N / 128) * T.c0;
      S.so = (uint32_t)(T.nb * 2 + (lane & 1)) * (uint32_t)T.nch * 4u;
    } else {
      S.sb = p.xts + (int64_t)p.F * T.c0;
      S.so = 0u;
    }
    return S;
  };

  Tile cur{}, nxt{};
  Src scur{}, snxt{};
  int nk_cur = 0, nk_nxt = 0;
  const uint32_t lds_base = lds_addr(lds);
  // issue ring step g = stage kt of the current tile, or stage kt - nk_cur of the next one
  // (clamped to its last stage: stages past the end re-read it into a slot that is not read)
  auto issue = [&](int g, int kt, bool even) {
    const bool in = kt < nk_cur;
    const int k = in ? kt : min(kt - nk_cur, nk_nxt - 1);
    const uint32_t st = lds_base + (uint32_t)((g & (TNST - 1)) * TSTAGE);
    const uint32_t kofs = (uint32_t)k * TBK;
    const uint8_t* A = (in ? scur.A : snxt.A) + kofs;
#pragma unroll
    for (int i = 0; i < 2; ++i) gload_lds16_s(A, in ? scur.aoff[i] : snxt.aoff[i], st + (wave_u * 2 + i) * 1024u);
    const uint8_t* B = (in ? scur.B : snxt.B) + kofs;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      gload_lds16_s(B, in ? scur.boff[i] : snxt.boff[i], st + (uint32_t)TA_BYTES + (wave_u * 2 + i) * 1024u);
    if (even) gload_lds4_s((in ? scur.sb : snxt.sb) + (k >> 1), in ? scur.so : snxt.so, st + (uint32_t)TS_OFF + wave_u * 256u);
  };

  const int frow = lane & 31, fhalf = lane >> 5;
  auto ld32 = [&](const char* base, int r) -> i32x8 {
    const u32x4 lo = *(const u32x4*)(base + t_off(r, 2 * fhalf));
    const u32x4 hi = *(const u32x4*)(base + t_off(r, 2 * fhalf + 1));
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  // rotating fragments (tgmm_fp8_kernel's schedule)
  i32x8 fr_a[TM], fr_b[2][TN];
  auto rd_a = [&](int g_, int i) -> i32x8 { return ld32(lds + (g_ & (TNST - 1)) * TSTAGE, wm * WTM + i * 32 + frow); };
  auto rd_b = [&](int g_, int j) -> i32x8 {
    return ld32(lds + (g_ & (TNST - 1)) * TSTAGE + TA_BYTES, wn * WTN + j * 32 + frow);
  };
  // scales of the chunk whose even stage sits in ring step g: the lane's four XT rows, the wave's GT block
  float sa_c[TM], sa_n[TM], sb_c = 0.0f, sb_n = 0.0f;
  auto read_scales = [&](int g, float* sa, float& sb) {
    const float* sc = (const float*)(lds + (g & (TNST - 1)) * TSTAGE + TS_OFF);
#pragma unroll
    for (int i = 0; i < TM; ++i) sa[i] = sc[wm * WTM + i * 32 + frow];
    sb = sc[256 + (wn >> 1)];
  };
  // P2: the same scales as E8M0 codes (the lane's four XT-row codes one per byte, opsel i)
  uint32_t ea_c = 0, ea_n = 0, eb_c = 0, eb_n = 0;
  auto read_codes = [&](int g, uint32_t& ea, uint32_t& eb) {
    const float* sc = (const float*)(lds + (g & (TNST - 1)) * TSTAGE + TS_OFF);
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) s |= e8m0_of(sc[wm * WTM + i * 32 + frow]) << (8 * i);
    ea = s;
    eb = e8m0_of(sc[256 + (wn >> 1)]);
  };
  auto mfma_p2 = [&](const i32x8& b, const i32x8& a, const f32x16& c, int i) -> f32x16 {
    switch (i) {
      case 0: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 0, (int)ea_c);
      case 1: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 1, (int)ea_c);
      case 2: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 2, (int)ea_c);
      default: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, (int)eb_c, 3, (int)ea_c);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // one stage: MFMAs of ring step g_ on fr_a / fr_b[cb] with step g_+1's fragments read in
  // between; at a chunk boundary (amax scales) each accumulator moves to the new chunk's units
  // one slot ahead of its MFMA
  auto rot_stage = [&](int g_, int cb, bool rescale, const float (&f)[TM]) {
#pragma unroll
    for (int j = 0; j < TN; ++j) fr_b[cb ^ 1][j] = rd_b(g_ + 1, j);
    auto rescale_acc = [&](int qq) {
      const int i = qq / TN, j = qq % TN;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] *= f[i];
    };
    if (rescale) rescale_acc(0);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (P2)
          acc[i][j] = mfma_p2(fr_b[cb][j], fr_a[i], acc[i][j], i);
        else
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fr_b[cb][j], fr_a[i], acc[i][j], 0, 0, 0, 127,
                                                                      0, 127);
        if (rescale && i * TN + j + 1 < TM * TN) rescale_acc(i * TN + j + 1);
      }
      fr_a[i] = rd_a(g_ + 1, i);
    }
  };
  int g = 0;
  // one chunk (an even and an odd stage); FIRST: the tile's first chunk (no rescale)
  auto kchunk = [&](int kb, auto first_tag) {
    constexpr bool FIRST = decltype(first_tag)::value;
    const int kt = 2 * kb;
    issue(g + TPD, kt + TPD, false);
    float f[TM] = {};
    if (FIRST) {
      rot_stage(g, 0, false, f);
    } else if (P2) {
      ea_c = ea_n;
      eb_c = eb_n;
      rot_stage(g, 0, false, f);
    } else {
      // (sa_c / sa_n) * (sb_c / sb_n): no product of two small scales is formed
      const float rb = sb_c * __builtin_amdgcn_rcpf(sb_n);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        f[i] = (sa_c[i] * __builtin_amdgcn_rcpf(sa_n[i])) * rb;
        sa_c[i] = sa_n[i];
      }
      sb_c = sb_n;
      rot_stage(g, 0, true, f);
    }
    // step g+2 landed (g+3 may be in flight); bare s_barrier (tgmm_fp8_kernel)
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS));
    __builtin_amdgcn_s_barrier();
    issue(g + 1 + TPD, kt + 1 + TPD, true);
    if constexpr (P2) read_codes(g + 2, ea_n, eb_n);  // the next chunk's codes (or the next tile's)
    else read_scales(g + 2, sa_n, sb_n);              // the next chunk's scales (or the next tile's)
    rot_stage(g + 1, 1, false, f);
    __builtin_amdgcn_s_waitcnt(MTX_VMCNT(LPS + 1));  // step g+3 landed (g+4 may be in flight)
    __builtin_amdgcn_s_barrier();
    g += 2;
  };
  // prologue of a ring that starts at tile cur: steps 0..2; 0 and 1 landed
  auto prologue = [&]() {
    g = 0;
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
  };
  // epilogue: scale (amax), stage through ring slot `slot` (32 rows x 64 bf16 columns per wave at
  // a time, 16-byte chunk c of row r at chunk c ^ (r & 7)) and store whole 128-byte row segments;
  // before the staging writes, every wave's fragment reads have completed (an LDS-only release
  // fence, then a barrier)
  auto epilogue = [&](int slot) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          acc[i][j][v] = P2 ? acc[i][j][v] : (acc[i][j][v] * sa_c[i]) * sb_c;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    char* wst = lds + slot * TSTAGE + wave * 4096;
    uint16_t* out = p.dw + (int64_t)cur.e * p.F * p.N + (int64_t)cur.fb * TBM * p.N + cur.nb * TBN;
    const uint32_t lo = (uint32_t)(wm * WTM + (lane >> 3)) * (uint32_t)p.N + (uint32_t)(wn * WTN + (lane & 7) * 8);
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
        *(u32x4*)(out + lo + (uint32_t)(i * 32 + rr * 8) * (uint32_t)p.N) = v;
      }
      __builtin_amdgcn_s_waitcnt(MTX_LGKMCNT0);  // reads done before the next block overwrites
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  };

  // ---- phase 1: experts of two or more chunks, the ring running across tiles ---------------------
  // ---- the zero tiles of the experts without rows (no LDS) ---------------------------------------
  for (int lid = total + (int)blockIdx.x; lid < all; lid += (int)gridDim.x) {
    const Tile T = decode(lid);
    uint16_t* out = p.dw + (int64_t)T.e * p.F * p.N + (int64_t)T.fb * TBM * p.N + T.nb * TBN;
    for (int i = tid; i < TBM * TBN / 8; i += 512) {
      const int r = i / (TBN / 8), cc = (i % (TBN / 8)) * 8;
      *(u32x4*)(out + (int64_t)r * p.N + cc) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  // ---- the tiles of the experts with rows ---------------------------------------------------------
  // The ring runs on from cur into nxt (chain) when both have two or more chunks: the three-stage
  // lookahead then stays within nxt.  Otherwise the lookahead re-reads cur's last stage into slots
  // that are not read, and the ring restarts at nxt with a prologue once those loads have landed.
  auto valid = [&](int jj) { return 8 * jj + xcd < total; };
  int j = q;
  if (valid(j)) {
    // the first tile is static and runs without lookahead; its epilogue draws two tickets (the
    // next tile and the one after), every later epilogue one (the tile after the next), so that a
    // workgroup holds at most one tile beyond the current one
    int j_next = -1;
    cur = decode(8 * j + xcd);
    scur = make_src(cur);
    nk_cur = 2 * cur.nch;
    snxt = scur;
    nk_nxt = nk_cur;
    bool chain = false;
    auto set_lookahead = [&]() {
      chain = valid(j_next) && cur.nch >= 2 && nxt.nch >= 2;
      if (chain) {
        snxt = make_src(nxt);
        nk_nxt = 2 * nxt.nch;
      } else {
        snxt = scur;
        nk_nxt = nk_cur;
      }
    };
    prologue();
    for (;;) {
      kchunk(0, std::true_type());
      for (int kb = 1; kb < cur.nch; ++kb) kchunk(kb, std::false_type());
      int tk = 0;
      if (wave_u == 0 && lane == 0)
        tk = lane_fetch_add(misc + 8 + xcd, j_next < 0 ? 2 : 1);
      // steps g .. g+2 (the next tile's first stages, or re-reads) are in flight; slot g-1 is free
      epilogue((g + TNST - 1) & (TNST - 1));
      if (wave_u == 0 && lane == 0) s_ticket = tk;
      __syncthreads();  // staging slot and s_ticket
      const int t = s_ticket;  // rewritten only in the next epilogue
      const bool first = j_next < 0;
      if (first) j_next = nx + t;
      const int j_after = first ? nx + t + 1 : nx + t;  // tickets rise, so j_next invalid => j_after too
      j = j_next;
      if (!valid(j)) break;
      const bool chained = chain;
      if (first) nxt = decode(8 * j + xcd);
      cur = nxt;
      nk_cur = 2 * cur.nch;
      scur = chained ? snxt : make_src(cur);
      j_next = j_after;
      if (valid(j_next)) nxt = decode(8 * j_next + xcd);
      set_lookahead();
      if (chained) {
        if constexpr (P2) {
          ea_c = ea_n;
          eb_c = eb_n;
        } else {
#pragma unroll
          for (int i = 0; i < TM; ++i) sa_c[i] = sa_n[i];
          sb_c = sb_n;
        }
      } else {
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

}  // namespace f8b

static inline int64_t fp8_grouped_chunks(int64_t M, int64_t E) { return ceil_div(M, 128) + E; }

}  // namespace mtx

using namespace mtx;

template <bool P2>
static int quant_weights_t_entry(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout, uint8_t* w_qt,
                                 float* w_scale_t, void* stream) {
  if (E < 0 || Kin < 0 || Kout < 0 || Kin % 128 || Kout % 128 || (dtype != MTX_F32 && dtype != MTX_BF16))
    return MTX_ERR_ARG;
  if (E == 0 || Kin == 0 || Kout == 0) return MTX_OK;
  if (!w || !w_qt || !w_scale_t) return MTX_ERR_ARG;
  if (((uintptr_t)w | (uintptr_t)w_qt) % 16) return MTX_ERR_ARG;  // 16-byte loads, 8-byte stores
  if (E > 65535 || Kin / 128 > 65535) return MTX_ERR_UNSUPPORTED;
  dim3 grid((unsigned)(Kout / 128), (unsigned)(Kin / 128), (unsigned)E);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MTX_F32)
    hipLaunchKernelGGL((f8b::quant_weights_t_kernel<float, P2>), grid, dim3(256), 0, st, (const float*)w, Kin, Kout,
                       w_qt, w_scale_t);
  else
    hipLaunchKernelGGL((f8b::quant_weights_t_kernel<uint16_t, P2>), grid, dim3(256), 0, st, (const uint16_t*)w, Kin,
                       Kout, w_qt, w_scale_t);
  return check_launch();
}

extern "C" int mtx_quant_fp8_weights_t(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout, uint8_t* w_qt,
                                       float* w_scale_t, void* stream) {
  return quant_weights_t_entry<false>(w, dtype, E, Kin, Kout, w_qt, w_scale_t, stream);
}

extern "C" int mtx_quant_fp8_weights_t_p2(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout,
                                          uint8_t* w_qt, float* w_scale_t, void* stream) {
  return quant_weights_t_entry<true>(w, dtype, E, Kin, Kout, w_qt, w_scale_t, stream);
}

extern "C" int64_t mtx_fp8_grouped_chunks(int64_t M, int64_t E) {
  if (M < 0 || E < 1) return -1;
  return fp8_grouped_chunks(M, E);
}

extern "C" int64_t mtx_fp8_grouped_workspace_size(int64_t E) {
  if (E < 1) return -1;
  return round_up((3 * E + 2 + 24) * 4, 256);
}

// workspace: cb [E+1], off [E+1], order [E], misc [24] (ints)
static int grouped_prologue(const int32_t* gs, int64_t E, int64_t M, void* ws, hipStream_t st, int** cb, int** off,
                            int** order, int** misc = nullptr) {
  int* b = (int*)ws;
  *cb = b;
  *off = b + E + 1;
  *order = b + 2 * E + 2;
  int* m = b + 3 * E + 2;
  if (misc) *misc = m;
  hipLaunchKernelGGL(f8b::chunk_prologue_kernel, dim3(1), dim3(1024), 0, st, gs, (int)E, (int)M, *cb, *off, *order,
                     m);
  return check_launch();
}

template <bool P2>
static int quant_grouped_t_entry(const void* x, int dtype, const int32_t* group_sizes, int64_t M, int64_t F, int64_t E,
                                 int blocks, uint8_t* xt, float* xt_scale, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  if (M < 0 || M > INT32_MAX / 2 || F <= 0 || F % 128 || E < 1 || E > 1024) return MTX_ERR_ARG;
  if (dtype != MTX_F32 && dtype != MTX_BF16) return MTX_ERR_ARG;
  if (!workspace || workspace_bytes < mtx_fp8_grouped_workspace_size(E)) return MTX_ERR_WORKSPACE;
  if (!group_sizes || !xt || !xt_scale || (M > 0 && !x)) return MTX_ERR_ARG;
  if (((uintptr_t)xt | (uintptr_t)x) % 16) return MTX_ERR_ARG;  // 16-byte loads and stores
  const int64_t C = fp8_grouped_chunks(M, E);
  if (C > 2147483647 / 128 || F / 128 > 65535) return MTX_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  int *cb, *off, *order;
  int rc = grouped_prologue(group_sizes, E, M, workspace, st, &cb, &off, &order);
  if (rc) return rc;
  dim3 grid((unsigned)C, (unsigned)(F / 128));
#define MTX_QG(T, B)                                                                                              \
  hipLaunchKernelGGL((f8b::quant_grouped_t_kernel<T, B, P2>), grid, dim3(256), 0, st, (const T*)x, (int)F, cb, off, \
                     (int)E, xt, xt_scale)
  if (dtype == MTX_F32) {
    if (blocks) MTX_QG(float, true); else MTX_QG(float, false);
  } else {
    if (blocks) MTX_QG(uint16_t, true); else MTX_QG(uint16_t, false);
  }
#undef MTX_QG
  return check_launch();
}

extern "C" int mtx_quant_fp8_grouped_t(const void* x, int dtype, const int32_t* group_sizes, int64_t M, int64_t F,
                                       int64_t E, int blocks, uint8_t* xt, float* xt_scale, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  return quant_grouped_t_entry<false>(x, dtype, group_sizes, M, F, E, blocks, xt, xt_scale, workspace,
                                      workspace_bytes, stream);
}

extern "C" int mtx_quant_fp8_grouped_t_p2(const void* x, int dtype, const int32_t* group_sizes, int64_t M, int64_t F,
                                          int64_t E, int blocks, uint8_t* xt, float* xt_scale, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  return quant_grouped_t_entry<true>(x, dtype, group_sizes, M, F, E, blocks, xt, xt_scale, workspace,
                                     workspace_bytes, stream);
}

static int tgmm_fp8_entry(bool p2, const uint8_t* xt, const float* xt_scale, const uint8_t* gt,
                          const float* gt_scale, const int32_t* group_sizes, int64_t M, int64_t F, int64_t N, int64_t E,
                          void* dw, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || M > INT32_MAX / 2 || F <= 0 || N <= 0 || E < 1 || E > 1024) return MTX_ERR_ARG;
  if (F % 128 || N % 128) return MTX_ERR_ARG;
  if (F % 256 || N % 256) return MTX_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < mtx_fp8_grouped_workspace_size(E)) return MTX_ERR_WORKSPACE;
  if (!xt || !xt_scale || !gt || !gt_scale || !group_sizes || !dw) return MTX_ERR_ARG;
  if (((uintptr_t)xt | (uintptr_t)gt) % 16) return MTX_ERR_ARG;
  const int64_t C = fp8_grouped_chunks(M, E);
  if ((F > N ? F : N) * C * 128 >= (int64_t(1) << 32)) return MTX_ERR_UNSUPPORTED;  // 32-bit byte offsets
  hipStream_t st = (hipStream_t)stream;
  int *cb, *off, *order, *misc;
  int rc = grouped_prologue(group_sizes, E, M, workspace, st, &cb, &off, &order, &misc);
  if (rc) return rc;
  f8b::TArgs a;
  a.xt = xt;
  a.xts = xt_scale;
  a.gt = gt;
  a.gts = gt_scale;
  a.dw = (uint16_t*)dw;
  a.cb = cb;
  a.order = order;
  a.E = (int)E;
  a.F = (int)F;
  a.N = (int)N;
  // XCD rectangles of the tile grid: xa x xb = 8 with xa | nf, xb | nn, fewest blocks per XCD
  const int nf = (int)(F / 256), nn = (int)(N / 256);
  a.xa = a.xb = 0;
  int best = 1 << 30;
  for (int xa = 1; xa <= 8; xa *= 2) {
    const int xb = 8 / xa;
    if (nf % xa || nn % xb) continue;
    const int blocks = nf / xa + nn / xb;
    if (blocks < best) {
      best = blocks;
      a.xa = xa;
      a.xb = xb;
    }
  }
  const int64_t tiles = E * (F / 256) * (N / 256);
#ifndef MTX_TGMM_PERSISTENT
#define MTX_TGMM_PERSISTENT 1
#endif
  // one workgroup per CU (a multiple of the 8 XCDs); with fewer than 8 tiles per workgroup the
  // tickets drawn a tile ahead leave the last tiles on few workgroups: the per-tile kernel then
  const int ncu = device_cu_count();
  const int64_t pgrid = ncu > 0 ? round_up(ncu, 8) : 256;
  if (MTX_TGMM_PERSISTENT && tiles >= 8 * pgrid) {
    const int64_t grid = pgrid;
    if (p2) hipLaunchKernelGGL(f8b::tgmm_fp8_p_kernel<true>, dim3((unsigned)grid), dim3(512), 0, st, a, misc);
    else hipLaunchKernelGGL(f8b::tgmm_fp8_p_kernel<false>, dim3((unsigned)grid), dim3(512), 0, st, a, misc);
    return check_launch();
  }
  const int64_t grid = round_up(tiles, 8);
  if (p2) hipLaunchKernelGGL(f8b::tgmm_fp8_kernel<true>, dim3((unsigned)grid), dim3(512), 0, st, a);
  else hipLaunchKernelGGL(f8b::tgmm_fp8_kernel<false>, dim3((unsigned)grid), dim3(512), 0, st, a);
  return check_launch();
}

extern "C" int mtx_tgmm_fp8(const uint8_t* xt, const float* xt_scale, const uint8_t* gt, const float* gt_scale,
                            const int32_t* group_sizes, int64_t M, int64_t F, int64_t N, int64_t E, void* dw,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  return tgmm_fp8_entry(false, xt, xt_scale, gt, gt_scale, group_sizes, M, F, N, E, dw, workspace, workspace_bytes,
                        stream);
}

extern "C" int mtx_tgmm_fp8_p2(const uint8_t* xt, const float* xt_scale, const uint8_t* gt, const float* gt_scale,
                               const int32_t* group_sizes, int64_t M, int64_t F, int64_t N, int64_t E, void* dw,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  return tgmm_fp8_entry(true, xt, xt_scale, gt, gt_scale, group_sizes, M, F, N, E, dw, workspace, workspace_bytes,
                        stream);
}

extern "C" int mtx_gmm_fp8_dlhs(const uint8_t* gq, const float* g_scale, const uint8_t* w_qt, const float* w_scale_t,
                                const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* dx,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  // dX [M, Kin] = dY [M, Kout] @ W[e]^T: the forward product with the weight codes in W's own
  // layout [E, Kin, Kout] (rows = output columns, k-contiguous over the reduction Kout)
  return mtx_gmm_fp8(gq, g_scale, w_qt, w_scale_t, group_sizes, M, Kout, Kin, E, dx, workspace, workspace_bytes,
                     stream);
}

extern "C" int mtx_gmm_fp8_dlhs_p2(const uint8_t* gq, const float* g_scale, const uint8_t* w_qt,
                                   const float* w_scale_t, const int32_t* group_sizes, int64_t M, int64_t Kin,
                                   int64_t Kout, int64_t E, void* dx, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  return mtx_gmm_fp8_p2(gq, g_scale, w_qt, w_scale_t, group_sizes, M, Kout, Kin, E, dx, workspace, workspace_bytes,
                        stream);
}
