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

  float sel[V], pay[V];
  bool ok[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = li + L * v;
    ok[v] = tok_ok && e < E;
    float x = ok[v] ? load_as_f32(logits, t * E + e, ldt) : -INFINITY;
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
    for (int off = 1; off < L; off <<= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      const float os = __shfl_xor(bs, off);
      if (cand_better(ov, oi, bv, bi)) { bv = ov; bi = oi; bs = os; }
    }
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
    for (int off = 1; off < L; off <<= 1) part += __shfl_xor(part, off);
    full_den = part;
    float ek = mine ? expf(my_s - lmax) : 0.0f;
    float den;
    if (norm) {
      den = ek;
      for (int off = 1; off < L; off <<= 1) den += __shfl_xor(den, off);
    } else {
      den = full_den;
    }
    w = ek / den;
  } else {
    float wk = mine ? my_s : 0.0f;
    if (norm) {
      float den = wk;
      for (int off = 1; off < L; off <<= 1) den += __shfl_xor(den, off);
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

}  // namespace mtx

using namespace mtx;

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
  int P = 1;
  while (P < E) P <<= 1;
  int L = P / 8 < 1 ? 1 : P / 8;
  while (L < K) L <<= 1;  // lane li < K of a token holds the round-li winner (K <= 64)
  if (L > 64) L = 64;
  const int V = (int)ceil_div(E, L);
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
