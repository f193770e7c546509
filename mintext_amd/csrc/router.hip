// Router top-k for the MoE layer on gfx950.
//
// One token is owned by a group of L = clamp(max(pow2ceil(E)/8, K), 1, 64) lanes of a wave; each lane
// holds V = ceil(E/L) <= 16 candidates (expert e = lane_in_group + L*v, so the logits row is
// read in L-wide runs).  Top-K is K rounds of a lane-group arg-max butterfly on
// (value, expert id) with ties going to the lower id, the order lax.top_k returns.
//
// Semantics (bzantium/mintext):
//   SIGMOID_GROUP follows MoERouter.__call__ / _group_topk_routing,
//   mintext/modules/moe.py:52-67 (sigmoid, + e_score_correction_bias, norm, scaling) and
//   moe.py:69-103 (top-2 sum per group, top-k groups, -inf mask, top-k, gather unbiased).
//   SOFTMAX has no counterpart in the reference; it is the Mixtral/Qwen3 router
//   (softmax in f32, top-k, renormalise over the top-k), selecting on the logits, which
//   orders experts exactly as the softmax probabilities do up to rounding ties.
#include "common.h"

namespace mtx {

struct Cand {
  float v;   // selection value
  int i;     // expert id, INT32_MAX = no candidate
  float s;   // payload: unbiased score (sigmoid mode) / logit (softmax mode)
};

__device__ __forceinline__ bool cand_better(float av, int ai, float bv, int bi) {
  if (ai == INT32_MAX) return false;
  if (bi == INT32_MAX) return true;
  return av > bv || (av == bv && ai < bi);
}

// Arg-max of (value, id, payload) over the token's L lanes (L a power of two <= 64).
template <int S = 0>
__device__ __forceinline__ void group_argmax(float& bv, int& bi, float& bs, int L) {
  if constexpr (S < 6) {
    if ((1 << S) < L) {
      const float ov = lane_xchg<S>(bv);
      const int oi = lane_xchg<S>(bi);
      const float os = lane_xchg<S>(bs);
      if (cand_better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
        bs = os;
      }
      group_argmax<S + 1>(bv, bi, bs, L);
    }
  }
}
// Sum over the token's L lanes (the same additions as an xor butterfly).
template <int S = 0>
__device__ __forceinline__ float group_sum(float x, int L) {
  if constexpr (S < 6) {
    if ((1 << S) < L) return group_sum<S + 1>(x + lane_xchg<S>(x), L);
  }
  return x;
}

// Selection for one token t owned by lanes li = 0..L-1 of its lane group (tok_local: the
// token's slot in the workgroup, for the group-limited scratch in smem).  load(e) returns the
// token's logit of expert e as f32.  Every thread of the workgroup must call it (the
// group-limited path synchronises the workgroup).
template <int V, typename Load>
__device__ __forceinline__ void router_select(Load load, int64_t t, bool tok_ok, int tok_local, int li, int L,
                                              int E, int K, int scoring, const float* __restrict__ bias,
                                              int n_group, int topk_group, int norm, float rscale,
                                              int32_t* __restrict__ idx_out, float* __restrict__ w_out,
                                              float* __restrict__ scores_out, int ldo, int extra, float* smem) {
  float sel[V], pay[V];
  bool ok[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = li + L * v;
    ok[v] = tok_ok && e < E;
    float x = ok[v] ? load(e) : -INFINITY;
    if (scoring == MTX_SCORING_SIGMOID_GROUP) {
      const float s = 1.0f / (1.0f + expf(-x));
      pay[v] = s;
      sel[v] = ok[v] ? s + (bias ? bias[e] : 0.0f) : -INFINITY;
    } else {
      pay[v] = x;
      sel[v] = x;
    }
  }

  // ---- group-limited masking (moe.py:76-95) --------------------------------------------
  if (scoring == MTX_SCORING_SIGMOID_GROUP && n_group > 1 && topk_group < n_group) {
    const int epg = E / n_group;
    float* rs = smem + tok_local * (E + 2 * n_group);
    float* gsc = rs + E;
    float* gsel = gsc + n_group;
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ok[v]) rs[li + L * v] = sel[v];
    __syncthreads();
    if (tok_ok) {
      for (int g = li; g < n_group; g += L) {
        float m1 = -INFINITY, m2 = -INFINITY;
        for (int j = 0; j < epg; ++j) {
          const float x = rs[g * epg + j];
          if (x > m1) { m2 = m1; m1 = x; }
          else if (x > m2) { m2 = x; }
        }
        gsc[g] = (epg >= 2) ? (m1 + m2) : m1;
      }
    }
    __syncthreads();
    if (tok_ok) {
      for (int g = li; g < n_group; g += L) {
        const float me = gsc[g];
        int rank = 0;
        for (int h = 0; h < n_group; ++h) {
          const float o = gsc[h];
          rank += (o > me || (o == me && h < g)) ? 1 : 0;
        }
        gsel[g] = (rank < topk_group) ? 1.0f : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e = li + L * v;
      if (ok[v] && gsel[e / epg] == 0.0f) sel[v] = -INFINITY;
    }
  }

  // ---- top-K: K rounds of lane-group arg-max --------------------------------------------
  bool taken[V];
#pragma unroll
  for (int v = 0; v < V; ++v) taken[v] = false;
  float my_v = -INFINITY, my_s = 0.0f, lmax = 0.0f;
  int my_i = INT32_MAX;
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY, bs = 0.0f;
    int bi = INT32_MAX;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e = li + L * v;
      if (ok[v] && !taken[v] && cand_better(sel[v], e, bv, bi)) { bv = sel[v]; bi = e; bs = pay[v]; }
    }
    group_argmax(bv, bi, bs, L);
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (li + L * v == bi) taken[v] = true;
    if (k == 0) lmax = bs;
    if (li == k) { my_v = bv; my_i = bi; my_s = bs; }
  }

  // ---- weights ---------------------------------------------------------------------------
  const bool mine = (li < K) && (my_i != INT32_MAX);
  float w;
  float full_den = 1.0f;
  if (scoring == MTX_SCORING_SOFTMAX) {
    float part = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ok[v]) part += expf(pay[v] - lmax);
    part = group_sum(part, L);
    full_den = part;
    float ek = mine ? expf(my_s - lmax) : 0.0f;
    float den;
    if (norm) {
      den = group_sum(ek, L);
    } else {
      den = full_den;
    }
    w = ek / den;
  } else {
    float wk = mine ? my_s : 0.0f;
    if (norm) {
      const float den = group_sum(wk, L);
      wk = wk / (den + 1e-20f);
    }
    w = wk;
  }
  w = w * rscale;
  (void)my_v;
  if (tok_ok && li < K) {
    idx_out[t * ldo + li] = my_i;
    w_out[t * ldo + li] = w;
  }
  // always-routed extra expert (a folded shared expert) in column K with weight 1
  if (tok_ok && extra >= 0 && li == 0) {
    idx_out[t * ldo + K] = extra;
    w_out[t * ldo + K] = 1.0f;
  }
  if (scores_out != nullptr) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (!ok[v]) continue;
      const int e = li + L * v;
      scores_out[t * E + e] = (scoring == MTX_SCORING_SOFTMAX) ? expf(pay[v] - lmax) / full_den : pay[v];
    }
  }
}

template <int V>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const void* __restrict__ logits, int ldt, int T, int E, int K, int L,
    int scoring, const float* __restrict__ bias, int n_group, int topk_group, int norm,
    float rscale, int32_t* __restrict__ idx_out, float* __restrict__ w_out,
    float* __restrict__ scores_out, int ldo, int extra) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tpw = 64 / L;
  const int li = lane % L;
  const int tok_local = wave * tpw + lane / L;
  const int tpb = (blockDim.x >> 6) * tpw;
  const int64_t t = (int64_t)blockIdx.x * tpb + tok_local;
  const bool tok_ok = t < T;
  router_select<V>([&](int e) { return load_as_f32(logits, t * E + e, ldt); }, t, tok_ok, tok_local, li, L, E, K,
                   scoring, bias, n_group, topk_group, norm, rscale, idx_out, w_out, scores_out, ldo, extra, smem);
}

// ---- router gate GEMM fused with the top-k ---------------------------------------------------
// logits = round_to_bf16(x @ Wg) (f32 accumulation), then router_select on those logits: the gate
// Linear.__call__ (mintext/modules/linear.py:123-147, bf16 dot with one rounding) feeding
// MoERouter (moe.py:41-103) without the [T,E] round trip.  A workgroup owns 32 tokens and all
// (up to 256) experts; its 4 waves split the reduction over D in quarters, each with
// v_mfma_f32_32x32x16_bf16 on operands loaded straight from memory (x rows and the gate weight
// in the nn.Linear layout wt [E,D] are both k-contiguous: one 16-byte load per lane and
// operand), and the quarters are added in wave order in LDS, so the sums are deterministic.
typedef __attribute__((ext_vector_type(8))) __bf16 gate_bf16x8;
typedef __attribute__((ext_vector_type(16))) float gate_f32x16;
constexpr int kGateTokens = 32;

template <int EB, int V>
__global__ __launch_bounds__(256) void gate_topk_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wt, int T, int D, int E, int K, int L, int scoring,
    const float* __restrict__ bias, int n_group, int topk_group, int norm, float rscale,
    int32_t* __restrict__ idx_out, float* __restrict__ w_out, uint16_t* __restrict__ logits_out,
    float* __restrict__ scores_out, int ldo, int extra) {
  constexpr int EP = EB * 32, LDP = EP + 1;  // logits tile row stride (+1: conflict-free)
  extern __shared__ float smem[];
  float* lg = smem;                              // [32][LDP] f32
  float* scratch = smem + kGateTokens * LDP;     // group-limited scratch of router_select
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kGateTokens;

  // ---- logits: wave w reduces k in [w*D/4, (w+1)*D/4) ------------------------------------
  gate_f32x16 acc[EB];
#pragma unroll
  for (int b = 0; b < EB; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
  const int r = lane & 31, kh = lane >> 5;
  const int64_t trow = min(t0 + r, (int64_t)T - 1);  // rows past T: computed, never stored
  const uint16_t* xa = x + trow * D + kh * 8;
  const uint16_t* wb[EB];
#pragma unroll
  for (int b = 0; b < EB; ++b) wb[b] = wt + (int64_t)min(b * 32 + r, E - 1) * D + kh * 8;
  const int kq = D / 4, kbeg = wave * kq;
#pragma unroll 4
  for (int k = kbeg; k < kbeg + kq; k += 16) {
    const gate_bf16x8 a = *(const gate_bf16x8*)(xa + k);
#pragma unroll
    for (int b = 0; b < EB; ++b) {
      const gate_bf16x8 w = *(const gate_bf16x8*)(wb[b] + k);
      acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, a, acc[b], 0, 0, 0);
    }
  }
  // lane l holds, for value 4g+q of block b, expert b*32 + 8g + 4(l/32) + q of token l%32
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int b = 0; b < EB; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float* dst = lg + r * LDP + b * 32 + 8 * g + 4 * kh + q;
            *dst = (w == 0) ? acc[b][4 * g + q] : *dst + acc[b][4 * g + q];
          }
    }
    __syncthreads();
  }
  // the gate output in the compute dtype (one rounding, as the reference's bf16 dot)
  for (int i = tid; i < kGateTokens * E; i += blockDim.x) {
    const int tt = i / E, e = i - tt * E;
    const uint16_t hb = f32_to_bf16(lg[tt * LDP + e]);
    lg[tt * LDP + e] = bf16_to_f32(hb);
    if (logits_out && t0 + tt < T) logits_out[(t0 + tt) * E + e] = hb;
  }
  __syncthreads();

  // ---- top-k of the tile's tokens (passes of 4 * 64/L tokens) ------------------------------
  const int tpw = 64 / L, li = lane % L, tpb = 4 * tpw;
  for (int p0 = 0; p0 < kGateTokens; p0 += tpb) {
    const int slot = wave * tpw + lane / L;
    const int tl = p0 + slot;
    const int64_t t = t0 + tl;
    const bool tok_ok = tl < kGateTokens && t < T;
    const float* row = lg + (tok_ok ? tl : 0) * LDP;
    router_select<V>([&](int e) { return row[e]; }, t, tok_ok, slot, li, L, E, K, scoring, bias, n_group, topk_group,
                     norm, rscale, idx_out, w_out, scores_out, ldo, extra, scratch);
    __syncthreads();  // the scratch of the next pass
  }
}

// ---- router VJP --------------------------------------------------------------------------
// d logits of the weights (and optionally of the scores) the forward returned, for fixed
// indices: the selection (top-k, group mask) carries no gradient and neither does the bias,
// which MoERouter keeps as a non-trainable variable (moe.py:37-39).  One wave per token.
//   SIGMOID_GROUP (moe.py:53,63-66,101): w_k = c * s_k / (S + 1e-20) with S = sum_j s_j
//     (c = routed_scaling_factor; w_k = c * s_k without norm), s = sigmoid(l), so
//     ds_k = c * (g_k - sum_j g_j s_j / (S + 1e-20)) / (S + 1e-20)  and  dl = ds * s * (1 - s).
//   SOFTMAX, norm: w = c * softmax over the selected logits, dl_{i_k} = c * u_k (g_k - sum_j u_j g_j)
//     with u = w / c; unselected logits get no gradient.  Without norm w_k = c * p_{i_k} of the
//     full softmax p, dl_e = c * p_e (g'_e - sum_k g_k p_{i_k}) with g'_e = g_k where e = i_k.
//   scores (sigmoid or full softmax) add dscores * s (1 - s), or p * (dscores - sum_j dscores_j p_j).
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}

__global__ __launch_bounds__(256) void router_topk_bwd_kernel(
    const void* __restrict__ logits, int ldt, int T, int E, int K, int scoring, int norm, float rscale,
    const int32_t* __restrict__ idx, int ldi, const float* __restrict__ dw, const float* __restrict__ dscores,
    void* __restrict__ dlogits, int dldt) {
  __shared__ int sel_e[4][64];
  __shared__ float sel_d[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t >= T) return;  // whole waves only: no workgroup barrier below
  const int64_t row = t * E;
  // the K selected experts and their upstream gradients, one per lane
  const bool kl = lane < K;
  const int ek = kl ? idx[t * ldi + lane] : -1;
  const bool kv = kl && ek >= 0 && ek < E;
  const float lk = kv ? load_as_f32(logits, row + ek, ldt) : 0.0f;
  const float gk = (kv && dw) ? dw[t * K + lane] : 0.0f;
  float dk = 0.0f;  // d logit of expert ek from the weights
  float pmax = 0.0f, pden = 1.0f, pdot = 0.0f;  // full-softmax terms
  if (scoring == MTX_SCORING_SIGMOID_GROUP) {
    const float s = kv ? 1.0f / (1.0f + expf(-lk)) : 0.0f;
    float ds;
    if (norm) {
      const float den = wave_sum(s) + 1e-20f;
      const float gs = wave_sum(gk * s);
      ds = rscale * (gk - gs / den) / den;
    } else {
      ds = rscale * gk;
    }
    dk = ds * s * (1.0f - s);
  } else {
    // the logit maximum over all experts (the top-1 logit) and the full softmax denominator
    float m = -INFINITY;
    for (int e = lane; e < E; e += 64) m = fmaxf(m, load_as_f32(logits, row + e, ldt));
    pmax = wave_max(m);
    const float ekx = kv ? expf(lk - pmax) : 0.0f;
    if (norm) {
      const float den = wave_sum(ekx);
      const float u = ekx / den;
      const float gu = wave_sum(gk * u);
      dk = rscale * u * (gk - gu);
    } else {
      float part = 0.0f;
      for (int e = lane; e < E; e += 64) part += expf(load_as_f32(logits, row + e, ldt) - pmax);
      pden = wave_sum(part);
      const float p = ekx / pden;
      pdot = wave_sum(gk * p);
      dk = rscale * p * gk;  // the -p_e * sum term is added per expert below
    }
  }
  if (kl) {
    sel_e[wave][lane] = kv ? ek : -1;
    sel_d[wave][lane] = dk;
  }
  float sdot = 0.0f;  // sum_j dscores_j p_j of the full softmax
  if (dscores && scoring == MTX_SCORING_SOFTMAX) {
    if (norm) {  // the full-softmax terms were not needed for the weights
      float m = -INFINITY;
      for (int e = lane; e < E; e += 64) m = fmaxf(m, load_as_f32(logits, row + e, ldt));
      pmax = wave_max(m);
      float part = 0.0f;
      for (int e = lane; e < E; e += 64) part += expf(load_as_f32(logits, row + e, ldt) - pmax);
      pden = wave_sum(part);
    }
    float part = 0.0f;
    for (int e = lane; e < E; e += 64)
      part += dscores[row + e] * (expf(load_as_f32(logits, row + e, ldt) - pmax) / pden);
    sdot = wave_sum(part);
  }
  __builtin_amdgcn_wave_barrier();
  for (int e = lane; e < E; e += 64) {
    float d = 0.0f;
    for (int k = 0; k < K; ++k)
      if (sel_e[wave][k] == e) d += sel_d[wave][k];
    if (scoring == MTX_SCORING_SOFTMAX && !norm && dw) {
      const float p = expf(load_as_f32(logits, row + e, ldt) - pmax) / pden;
      d -= rscale * p * pdot;
    }
    if (dscores) {
      const float l = load_as_f32(logits, row + e, ldt);
      if (scoring == MTX_SCORING_SIGMOID_GROUP) {
        const float s = 1.0f / (1.0f + expf(-l));
        d += dscores[row + e] * s * (1.0f - s);
      } else {
        const float p = expf(l - pmax) / pden;
        d += p * (dscores[row + e] - sdot);
      }
    }
    store_from_f32(dlogits, row + e, dldt, d);
  }
}

}  // namespace mtx

using namespace mtx;

static void router_lanes(int64_t E, int64_t K, int* L_out, int* V_out) {
  int P = 1;
  while (P < E) P <<= 1;
  int L = P / 8 < 1 ? 1 : P / 8;
  while (L < K) L <<= 1;  // lane li < K of a token holds the round-li winner (K <= 64)
  if (L > 64) L = 64;
  *L_out = L;
  *V_out = (int)ceil_div(E, L);
}

extern "C" int mtx_gate_router_topk(const void* x, int dtype, const void* gate_weight_t, int64_t T, int64_t D,
                                    int64_t E, int64_t K, int scoring, const float* bias, int64_t n_group,
                                    int64_t topk_group, int norm_topk_prob, float routed_scaling_factor,
                                    int64_t shared_expert, int32_t* topk_idx, float* topk_w, void* logits_out,
                                    float* scores, void* stream) {
  if (T < 0 || D < 0 || E < 1 || K < 1 || K > E || K > 64) return MTX_ERR_ARG;
  if (shared_expert >= 0 && (shared_expert < E || shared_expert > INT32_MAX)) return MTX_ERR_ARG;
  if (scoring != MTX_SCORING_SOFTMAX && scoring != MTX_SCORING_SIGMOID_GROUP) return MTX_ERR_ARG;
  if (n_group < 1) n_group = 1;
  if (topk_group < 1) topk_group = 1;
  if (scoring == MTX_SCORING_SIGMOID_GROUP && (E % n_group != 0 || topk_group > n_group)) return MTX_ERR_ARG;
  if (dtype != MTX_BF16 || E > 256 || D % 64 != 0 || D == 0) return MTX_ERR_UNSUPPORTED;
  if (T == 0) return MTX_OK;
  if (!x || !gate_weight_t || !topk_idx || !topk_w) return MTX_ERR_ARG;
  if ((uintptr_t)x % 16 != 0 || (uintptr_t)gate_weight_t % 16 != 0) return MTX_ERR_ARG;
  int L, V;
  router_lanes(E, K, &L, &V);
  const int EB = (int)ceil_div(E, 32), EBp = EB <= 1 ? 1 : EB <= 2 ? 2 : EB <= 4 ? 4 : 8;
  const int tpb = 4 * (64 / L);
  const size_t shm = ((size_t)kGateTokens * (EBp * 32 + 1) + (size_t)tpb * (size_t)(E + 2 * n_group)) * sizeof(float);
  const int grid = (int)ceil_div(T, kGateTokens);
  hipStream_t st = (hipStream_t)stream;
#define MTX_GATE(EBT, VV)                                                                                         \
  hipLaunchKernelGGL((gate_topk_kernel<EBT, VV>), dim3(grid), dim3(256), shm, st, (const uint16_t*)x,             \
                     (const uint16_t*)gate_weight_t, (int)T, (int)D, (int)E, (int)K, L, scoring, bias, (int)n_group, \
                     (int)topk_group, norm_topk_prob, routed_scaling_factor, topk_idx, topk_w, (uint16_t*)logits_out, scores, \
                     (int)(shared_expert >= 0 ? K + 1 : K), (int)(shared_expert >= 0 ? shared_expert : -1))
#define MTX_GATE_V(EBT)                      \
  if (V <= 1) MTX_GATE(EBT, 1);              \
  else if (V <= 2) MTX_GATE(EBT, 2);         \
  else if (V <= 4) MTX_GATE(EBT, 4);         \
  else MTX_GATE(EBT, 8);
  if (EBp == 1) { MTX_GATE_V(1) }
  else if (EBp == 2) { MTX_GATE_V(2) }
  else if (EBp == 4) { MTX_GATE_V(4) }
  else { MTX_GATE_V(8) }
#undef MTX_GATE_V
#undef MTX_GATE
  return check_launch();
}

static int router_launch(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K, int scoring,
                         const float* bias, int64_t n_group, int64_t topk_group, int norm_topk_prob,
                         float routed_scaling_factor, int32_t* topk_idx, float* topk_w, float* scores, int64_t ldo,
                         int64_t extra, void* stream) {
  if (T < 0 || E < 1 || E > 1024 || K < 1 || K > E || K > 64) return MTX_ERR_ARG;
  if (logits_dtype != MTX_F32 && logits_dtype != MTX_BF16) return MTX_ERR_ARG;
  if (scoring != MTX_SCORING_SOFTMAX && scoring != MTX_SCORING_SIGMOID_GROUP) return MTX_ERR_ARG;
  if (n_group < 1) n_group = 1;
  if (topk_group < 1) topk_group = 1;
  if (scoring == MTX_SCORING_SIGMOID_GROUP && (E % n_group != 0 || topk_group > n_group)) return MTX_ERR_ARG;
  if (T == 0) return MTX_OK;
  if (!logits || !topk_idx || !topk_w) return MTX_ERR_ARG;
  // L lanes per token with up to 8 candidates each: few butterfly steps per round and several
  // tokens per wave (E = 8: one lane per token; E = 128: 16 lanes; E >= 512: 64 lanes)
  int L, V;
  router_lanes(E, K, &L, &V);
  const int tpb = 4 * (64 / L);
  const int grid = (int)ceil_div(T, tpb);
  size_t shm = 0;
  if (scoring == MTX_SCORING_SIGMOID_GROUP && n_group > 1 && topk_group < n_group)
    shm = (size_t)tpb * (size_t)(E + 2 * n_group) * sizeof(float);
  hipStream_t st = (hipStream_t)stream;
#define MTX_LAUNCH_TOPK(VV)                                                                      \
  hipLaunchKernelGGL(router_topk_kernel<VV>, dim3(grid), dim3(256), shm, st, logits, logits_dtype, \
                     (int)T, (int)E, (int)K, L, scoring, bias, (int)n_group, (int)topk_group,      \
                     norm_topk_prob, routed_scaling_factor, topk_idx, topk_w, scores, (int)ldo, (int)extra)
  if (V <= 1) MTX_LAUNCH_TOPK(1);
  else if (V <= 2) MTX_LAUNCH_TOPK(2);
  else if (V <= 4) MTX_LAUNCH_TOPK(4);
  else if (V <= 8) MTX_LAUNCH_TOPK(8);
  else MTX_LAUNCH_TOPK(16);
#undef MTX_LAUNCH_TOPK
  return check_launch();
}

extern "C" int mtx_router_topk(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                               int scoring, const float* bias, int64_t n_group, int64_t topk_group,
                               int norm_topk_prob, float routed_scaling_factor,
                               int32_t* topk_idx, float* topk_w, float* scores, void* stream) {
  return router_launch(logits, logits_dtype, T, E, K, scoring, bias, n_group, topk_group, norm_topk_prob,
                       routed_scaling_factor, topk_idx, topk_w, scores, K, -1, stream);
}

extern "C" int mtx_router_topk_shared(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                                      int scoring, const float* bias, int64_t n_group, int64_t topk_group,
                                      int norm_topk_prob, float routed_scaling_factor, int64_t shared_expert,
                                      int32_t* topk_idx, float* topk_w, float* scores, void* stream) {
  if (shared_expert < E || shared_expert > INT32_MAX) return MTX_ERR_ARG;
  return router_launch(logits, logits_dtype, T, E, K, scoring, bias, n_group, topk_group, norm_topk_prob,
                       routed_scaling_factor, topk_idx, topk_w, scores, K + 1, shared_expert, stream);
}

extern "C" int mtx_router_topk_bwd(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                                   int scoring, int norm_topk_prob, float routed_scaling_factor,
                                   const int32_t* topk_idx, int64_t idx_ld, const float* d_topk_w,
                                   const float* d_scores, void* d_logits, int d_logits_dtype, void* stream) {
  if (T < 0 || E < 1 || K < 1 || K > E || K > 64 || idx_ld < K) return MTX_ERR_ARG;
  if (logits_dtype != MTX_F32 && logits_dtype != MTX_BF16) return MTX_ERR_ARG;
  if (d_logits_dtype != MTX_F32 && d_logits_dtype != MTX_BF16) return MTX_ERR_ARG;
  if (scoring != MTX_SCORING_SOFTMAX && scoring != MTX_SCORING_SIGMOID_GROUP) return MTX_ERR_ARG;
  if (T == 0) return MTX_OK;
  if (!logits || !topk_idx || !d_logits) return MTX_ERR_ARG;
  if (T > INT32_MAX) return MTX_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(router_topk_bwd_kernel, dim3((unsigned)ceil_div(T, 4)), dim3(256), 0, (hipStream_t)stream,
                     logits, logits_dtype, (int)T, (int)E, (int)K, scoring, norm_topk_prob, routed_scaling_factor,
                     topk_idx, (int)idx_ld, d_topk_w, d_scores, d_logits, d_logits_dtype);
  return check_launch();
}

// Loss-free load balancing (trainer.py:371-410 for one layer): bias[e] += rate * sign(mean - counts[e])
// with mean = float(sum(counts)) / float(E), one workgroup.
__global__ __launch_bounds__(1024) void expert_bias_update_kernel(const int32_t* __restrict__ counts, int E, float rate,
                                                                  float* __restrict__ bias) {
  __shared__ long long wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  long long part = 0;
  for (int e = tid; e < E; e += blockDim.x) part += counts[e];
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) wsum[w] = part;
  __syncthreads();
  long long total = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) total += wsum[i];
  const float mean = (float)total / (float)E;
  for (int e = tid; e < E; e += blockDim.x) {
    const float d = mean - (float)counts[e];
    const float sgn = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
    bias[e] = bias[e] + sgn * rate;
  }
}

extern "C" int mtx_expert_bias_update(const int32_t* expert_counts, int64_t E, float rate, float* bias,
                                      void* stream) {
  if (E < 1 || E > (int64_t(1) << 20)) return MTX_ERR_ARG;
  if (!expert_counts || !bias) return MTX_ERR_ARG;
  hipLaunchKernelGGL(expert_bias_update_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, expert_counts, (int)E,
                     rate, bias);
  return check_launch();
}
