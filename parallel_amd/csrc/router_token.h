// Per-token router arithmetic shared by the router kernels and the combine
// backward that finishes the router's top-k backward (the token layout, the
// reductions over a token's lanes, the softmax statistics, and one token's
// top-k backward).
//
// Reference arithmetic: TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267
// (router) and :514-593 (load_balancing_loss_func).
#pragma once

#include <type_traits>

#include "common.h"

namespace moe {

constexpr int kMaxPerLane = 16;  // E <= 1024
constexpr int kMaxTopK = 16;
constexpr int kRouterWaves = 4;  // waves per block

// Token layout.  A token occupies LPT consecutive lanes: one 16-lane DPP row
// (E <= 256, four tokens per wave) or the whole wave (E <= 1024).  Lane `sub`
// of a token holds experts sub, sub + LPT, ... (NPL of them, a power of two),
// so the softmax statistics and the k-way selection are reductions over the
// token's lanes with no LDS.  With 16-lane rows each reduction is 4 DPP steps
// serving 4 tokens at once; one token per wave spent about 850 VALU
// instructions per token, most of them in 6-step wave reductions.
// The kernels are instantiated per (LPT, NPL) and KT (top-k; 0 = any k up to
// kMaxTopK), so that the per-lane loops have fixed trip counts.  Items past E
// read as -inf and are never selected; the arithmetic is that of any NPL
// large enough for E.
template <int LPT>
struct Tok {
  static_assert(LPT == 16 || LPT == kWave, "a token is one DPP row or one wave");
  static constexpr int kPerBlock = kRouterWaves * (kWave / LPT);
  __device__ static int sub() { return threadIdx.x & (LPT - 1); }
  // The token's slot in the block (wave-major, then row).
  __device__ static int slot() { return threadIdx.x / LPT; }
};

// Reductions over a token's lanes.  Every lane of the token gets the result,
// bit for bit: each butterfly step combines a pair of lanes commutatively.
template <int LPT>
__device__ __forceinline__ float tok_max(float v) {
  if constexpr (LPT == kWave) {
    return wave_max(v);
  } else {
    v = fmaxf(v, dpp_move<dpp::kQuadXor1>(v, v));
    v = fmaxf(v, dpp_move<dpp::kQuadXor2>(v, v));
    v = fmaxf(v, dpp_move<dpp::kHalfMirror>(v, v));
    return fmaxf(v, dpp_move<dpp::kMirror>(v, v));
  }
}
template <int LPT>
__device__ __forceinline__ float tok_sum(float v) {
  if constexpr (LPT == kWave) {
    return wave_sum(v);
  } else {
    v += dpp_move<dpp::kQuadXor1>(0.0f, v);
    v += dpp_move<dpp::kQuadXor2>(0.0f, v);
    v += dpp_move<dpp::kHalfMirror>(0.0f, v);
    return v + dpp_move<dpp::kMirror>(0.0f, v);
  }
}
template <int LPT>
__device__ __forceinline__ void tok_argmax(float& v, int& i) {
  if constexpr (LPT == kWave) {
    wave_argmax(v, i);
  } else {
    argmax_step<dpp::kQuadXor1>(v, i);
    argmax_step<dpp::kQuadXor2>(v, i);
    argmax_step<dpp::kHalfMirror>(v, i);
    argmax_step<dpp::kMirror>(v, i);
  }
}

// Loads one token's logits; absent experts read as -inf.
template <int LPT, int NPL>
__device__ __forceinline__ void load_row(const float* row, int E, float (&v)[NPL]) {
  const int sub = Tok<LPT>::sub();
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    v[j] = e < E ? row[e] : -INFINITY;
  }
}

struct SoftmaxStats {
  float max, sum;
};

template <int LPT, int NPL>
__device__ __forceinline__ SoftmaxStats softmax_stats(const float (&v)[NPL]) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NPL; ++j) m = fmaxf(m, v[j]);
  m = tok_max<LPT>(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NPL; ++j)
    if (v[j] != -INFINITY) s += expf(v[j] - m);
  s = tok_sum<LPT>(s);
  return {m, s};
}

// One token's top-k backward: the renormalisation and softmax backward of
// its k selected scores and, with aux_stats, the aux loss's logits gradient
// (p_e (g_e - <g, p>), g_e = d_aux E w c_e / W^2), plus an added logits
// gradient.  It comes in two parts so that a caller can issue the token's
// loads ahead of other work: topk_bwd_load reads the token's logits, the
// added gradient, its selected experts and, with aux_stats, the aux terms'
// inputs; topk_bwd_finish (with_aux when aux_stats was given) forms d_logits
// from the selection's score gradients ds (selection order).  The result's
// arithmetic does not depend on where ds came from.
template <int LPT, int NPL, int KT>
struct TopkBwdRow {
  static constexpr int KM = KT ? KT : kMaxTopK;
  float v[NPL];    // the token's logits (-inf past E)
  float add[NPL];  // the added logits gradient (0 without one)
  int idx[KM];     // selected experts; -1 for an id outside [0, E)
  // With aux statistics: the experts' routed counts c_e, the weight total W,
  // the token's weight w and the aux loss's incoming gradient.
  float ce[NPL];
  float W, w, d_aux;
};

template <int LPT, int NPL, int KT>
__device__ __forceinline__ void topk_bwd_load(TopkBwdRow<LPT, NPL, KT>& r, const float* __restrict__ logits,
                                              const int64_t* __restrict__ indices, const float* d_add, int64_t t,
                                              int E, int k, const float* __restrict__ token_weight,
                                              const float* __restrict__ aux_stats, const float* __restrict__ d_aux) {
  const int sub = Tok<LPT>::sub();
  const int64_t base = t * E;
  load_row<LPT>(logits + base, E, r.v);
  // The added gradient is loaded with the logits, not after the arithmetic.
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    r.add[j] = (d_add && e < E) ? d_add[base + e] : 0.0f;
  }
#pragma unroll
  for (int q = 0; q < TopkBwdRow<LPT, NPL, KT>::KM; ++q) {
    r.idx[q] = -1;
    if (q < k) {
      const int64_t id = indices[t * k + q];
      r.idx[q] = (id >= 0 && id < E) ? static_cast<int>(id) : -1;
    }
  }
  r.W = r.d_aux = 0.0f;
  r.w = 1.0f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) r.ce[j] = 0.0f;
  if (aux_stats) {
    r.W = aux_stats[E];
    r.w = token_weight ? token_weight[t] : 1.0f;
    r.d_aux = d_aux[0];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int e = sub + j * LPT;
      if (e < E) r.ce[j] = aux_stats[e];
    }
  }
}

// d_logits = p (dp - <dp, p>) (+ the aux term, + the added gradient), dp
// scattered from the (renormalised) top-k; the fp32 result goes to d_logits
// and its bf16 rounding to d_logits_bf16 (either may be null).  With
// bf16_terms (bf16 logits, the router under bf16 autocast) every gradient
// term is a bf16 tensor's: ds, the softmax path's gradient and the aux term
// are rounded to bf16 and every sum is rounded again, as autograd sums a
// bf16 tensor's gradients.
template <int LPT, int NPL, int KT>
__device__ __forceinline__ void topk_bwd_finish(TopkBwdRow<LPT, NPL, KT>& r,
                                                float (&ds)[TopkBwdRow<LPT, NPL, KT>::KM],
                                                const float* __restrict__ logits, int64_t t, int E, int k, int norm,
                                                bool has_add, bool with_aux, float* d_logits,
                                                bf16_t* __restrict__ d_logits_bf16, int bf16_terms) {
  constexpr int KM = TopkBwdRow<LPT, NPL, KT>::KM;
  const int sub = Tok<LPT>::sub();
  const int64_t base = t * E;
  const SoftmaxStats st = softmax_stats<LPT>(r.v);
  const float inv_sum = 1.0f / st.sum;
  auto round_bf16 = [](float x) { return bf16_to_f32(f32_to_bf16(x)); };
  if (with_aux) {
    const float W = r.W;
    const float scale = r.d_aux * static_cast<float>(E) * r.w / (W * W);
    float p[NPL], g[NPL];
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int e = sub + j * LPT;
      p[j] = 0.0f;
      g[j] = 0.0f;
      if (e < E) {
        p[j] = expf(r.v[j] - st.max) * inv_sum;
        g[j] = scale * r.ce[j];
        dot += p[j] * g[j];
      }
    }
    dot = tok_sum<LPT>(dot);
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const float d = p[j] * (g[j] - dot);
      if (bf16_terms) {
        r.add[j] = has_add ? round_bf16(r.add[j] + round_bf16(d)) : round_bf16(d);
      } else {
        r.add[j] = has_add ? r.add[j] + d : d;
      }
    }
  }

  float pv[KM];
  float tot = 0.0f;
#pragma unroll
  for (int q = 0; q < KM; ++q) {
    if (q < k) {
      const bool ok = r.idx[q] >= 0;
      // bf16 logits come with bf16 scores, whose gradient is a bf16 tensor
      if (bf16_terms) ds[q] = round_bf16(ds[q]);
      float lv;
      if constexpr (LPT == kWave) {
        // One token per wave: the selected logit is already in lane e % 64
        // (v[e / 64]), fetched by readlane rather than a second load.
        const int e = __builtin_amdgcn_readfirstlane(ok ? r.idx[q] : 0);
        float cand = r.v[0];
#pragma unroll
        for (int j = 1; j < NPL; ++j) cand = (e / kWave == j) ? r.v[j] : cand;
        lv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cand), e & (kWave - 1)));
      } else {
        lv = ok ? logits[base + r.idx[q]] : 0.0f;
      }
      pv[q] = ok ? expf(lv - st.max) * inv_sum : 0.0f;
      tot += pv[q];
    }
  }
  // Renormalisation backward: s_r = v_r / V  ->  dv_r = (ds_r - sum_i ds_i s_i) / V.
  float dv[KM];
  if (norm) {
    float dot = 0.0f;
#pragma unroll
    for (int q = 0; q < KM; ++q)
      if (q < k) dot += ds[q] * (pv[q] / tot);
#pragma unroll
    for (int q = 0; q < KM; ++q)
      if (q < k) dv[q] = (ds[q] - dot) / tot;
  } else {
#pragma unroll
    for (int q = 0; q < KM; ++q)
      if (q < k) dv[q] = ds[q];
  }
  float c = 0.0f;  // <dp, p> = sum_r dv_r p_{idx_r}
#pragma unroll
  for (int q = 0; q < KM; ++q)
    if (q < k) c += dv[q] * pv[q];

#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    if (e < E) {
      float dp = 0.0f;
#pragma unroll
      for (int q = 0; q < KM; ++q)
        if (q < k && r.idx[q] == e) dp += dv[q];
      float p = expf(r.v[j] - st.max) * inv_sum;
      float g = p * (dp - c);
      if (bf16_terms) g = round_bf16(g);
      if (has_add || with_aux) g += r.add[j];
      if (d_logits) d_logits[base + e] = g;
      if (d_logits_bf16) d_logits_bf16[base + e] = f32_to_bf16(g);
    }
  }
}

// Instantiation for E experts: lanes per token, experts per lane rounded up
// to a power of two, and top-k k (the specialised k, or the generic 0).  The
// selecting kernels take 16 lanes per token up to 256 experts (their k rounds
// of reductions dominate); the backward kernels, which only stream a row in
// and out, keep one wave per token so that more waves hide their loads.
template <bool kWaveToken = false, class F>
void with_npl(int64_t E, F&& f) {
  using L16 = std::integral_constant<int, 16>;
  using L64 = std::integral_constant<int, kWave>;
  static_assert(16 * kMaxPerLane == 256, "E <= 256 fits 16 lanes per token");
  if constexpr (!kWaveToken) {
    if (E <= 256) {
      if (E <= 16) f(L16{}, std::integral_constant<int, 1>{});
      else if (E <= 32) f(L16{}, std::integral_constant<int, 2>{});
      else if (E <= 64) f(L16{}, std::integral_constant<int, 4>{});
      else if (E <= 128) f(L16{}, std::integral_constant<int, 8>{});
      else f(L16{}, std::integral_constant<int, 16>{});
      return;
    }
  }
  if (E <= 64) f(L64{}, std::integral_constant<int, 1>{});
  else if (E <= 128) f(L64{}, std::integral_constant<int, 2>{});
  else if (E <= 256) f(L64{}, std::integral_constant<int, 4>{});
  else if (E <= 512) f(L64{}, std::integral_constant<int, 8>{});
  else f(L64{}, std::integral_constant<int, 16>{});
}
template <bool kWaveToken = false, class F>
void with_npl_k(int64_t E, int64_t k, F&& f) {
  with_npl<kWaveToken>(E, [&](auto L, auto N) {
    switch (k) {
      case 1: f(L, N, std::integral_constant<int, 1>{}); break;
      case 2: f(L, N, std::integral_constant<int, 2>{}); break;
      case 4: f(L, N, std::integral_constant<int, 4>{}); break;
      case 6: f(L, N, std::integral_constant<int, 6>{}); break;
      case 8: f(L, N, std::integral_constant<int, 8>{}); break;
      default: f(L, N, std::integral_constant<int, 0>{}); break;
    }
  });
}

}  // namespace moe
