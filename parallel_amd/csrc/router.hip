// Router top-k softmax and the Switch load-balancing loss (gfx950).
//
// One 64-lane wave per token: lane l holds experts l, l+64, ... in registers,
// so softmax statistics and the k-way selection are wave reductions with no
// LDS.  Selection is on the logits (softmax is monotone), largest first, ties
// to the lower expert index; probabilities are exp(l - max) / sum in fp32.
//
// Reference arithmetic: TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267
// (router) and :514-593 (load_balancing_loss_func); the one-rank SP variant is
// parallel/parallel/engine/model_parallel/sequence_parallel.py:239-280.
#include "common.h"

namespace moe {

constexpr int kMaxPerLane = 16;  // E <= 1024
constexpr int kMaxTopK = 16;
constexpr int kRouterWaves = 4;  // waves per block

// Loads one token's logits; absent experts read as -inf.
__device__ __forceinline__ void load_row(const float* row, int E, float (&v)[kMaxPerLane], int npl) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    int e = lane + j * kWave;
    v[j] = (j < npl && e < E) ? row[e] : -INFINITY;
  }
}

struct SoftmaxStats {
  float max, sum;
};

__device__ __forceinline__ SoftmaxStats softmax_stats(const float (&v)[kMaxPerLane], int npl) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    if (j < npl) m = fmaxf(m, v[j]);
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    if (j < npl && v[j] != -INFINITY) s += expf(v[j] - m);
  s = wave_sum(s);
  return {m, s};
}

// k-way selection: sel_idx/sel_logit are wave-uniform after the call.
__device__ __forceinline__ void select_topk(const float (&v)[kMaxPerLane], int npl, int E, int k,
                                            int (&sel_idx)[kMaxTopK], float (&sel_logit)[kMaxTopK]) {
  const int lane = threadIdx.x & (kWave - 1);
  unsigned taken = 0;  // bit j: item j of this lane already selected
  for (int r = 0; r < k; ++r) {
    float best = -INFINITY;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      int e = lane + j * kWave;
      // Items are visited in increasing e, so ">" keeps the lower index on
      // ties; the first live item is always taken (covers -inf logits).
      if (j < npl && e < E && !(taken & (1u << j)) && (v[j] > best || bidx == 0x7fffffff)) {
        best = v[j];
        bidx = e;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      float ob = __shfl_xor(best, o, kWave);
      int oi = __shfl_xor(bidx, o, kWave);
      if (ob > best || (ob == best && oi < bidx)) {
        best = ob;
        bidx = oi;
      }
    }
    sel_idx[r] = bidx;
    sel_logit[r] = best;
    if (bidx != 0x7fffffff && (bidx & (kWave - 1)) == lane) taken |= 1u << (bidx / kWave);
  }
}

__global__ __launch_bounds__(kRouterWaves * kWave) void router_topk_fwd_kernel(const float* __restrict__ logits,
                                                                                float* __restrict__ scores,
                                                                                int64_t* __restrict__ indices, int T,
                                                                                int E, int k, int norm) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const int npl = (E + kWave - 1) / kWave;
  float v[kMaxPerLane];
  load_row(logits + static_cast<int64_t>(t) * E, E, v, npl);
  SoftmaxStats st = softmax_stats(v, npl);
  int sel[kMaxTopK];
  float sl[kMaxTopK];
  select_topk(v, npl, E, k, sel, sl);
  float pv[kMaxTopK];
  float tot = 0.0f;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r < k) {
      pv[r] = expf(sl[r] - st.max) / st.sum;
      tot += pv[r];
    }
  }
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r < k && lane == r) {
      scores[static_cast<int64_t>(t) * k + r] = norm ? pv[r] / tot : pv[r];
      indices[static_cast<int64_t>(t) * k + r] = sel[r];
    }
  }
}

// d_logits = p * (dp - <dp, p>), dp scattered from the (renormalised) top-k.
__global__ __launch_bounds__(kRouterWaves * kWave) void router_topk_bwd_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ indices, const float* __restrict__ d_scores, int T,
    int E, int k, int norm, float* __restrict__ d_logits, int accumulate, bf16_t* __restrict__ d_logits_bf16) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const int npl = (E + kWave - 1) / kWave;
  float v[kMaxPerLane];
  const float* row = logits + static_cast<int64_t>(t) * E;
  load_row(row, E, v, npl);
  SoftmaxStats st = softmax_stats(v, npl);
  const float inv_sum = 1.0f / st.sum;

  int idx[kMaxTopK];
  float pv[kMaxTopK], ds[kMaxTopK];
  float tot = 0.0f;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r < k) {
      int64_t id = indices[static_cast<int64_t>(t) * k + r];
      bool ok = id >= 0 && id < E;
      idx[r] = ok ? static_cast<int>(id) : -1;
      ds[r] = d_scores[static_cast<int64_t>(t) * k + r];
      pv[r] = ok ? expf(row[idx[r]] - st.max) * inv_sum : 0.0f;
      tot += pv[r];
    }
  }
  // Renormalisation backward: s_r = v_r / V  ->  dv_r = (ds_r - sum_i ds_i s_i) / V.
  float dv[kMaxTopK];
  if (norm) {
    float dot = 0.0f;
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r)
      if (r < k) dot += ds[r] * (pv[r] / tot);
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r)
      if (r < k) dv[r] = (ds[r] - dot) / tot;
  } else {
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r)
      if (r < k) dv[r] = ds[r];
  }
  float c = 0.0f;  // <dp, p> = sum_r dv_r p_{idx_r}
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r)
    if (r < k) c += dv[r] * pv[r];

  float* drow = d_logits + static_cast<int64_t>(t) * E;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    int e = lane + j * kWave;
    if (j < npl && e < E) {
      float dp = 0.0f;
#pragma unroll
      for (int r = 0; r < kMaxTopK; ++r)
        if (r < k && idx[r] == e) dp += dv[r];
      float p = expf(v[j] - st.max) * inv_sum;
      float g = p * (dp - c);
      if (accumulate) g += drow[e];
      drow[e] = g;
      if (d_logits_bf16) d_logits_bf16[static_cast<int64_t>(t) * E + e] = f32_to_bf16(g);
    }
  }
}

// ------------------------------------------------------------------ aux loss

constexpr int kAuxBlocksMax = 256;

int aux_blocks(int64_t T) {
  int64_t b = (T + 63) / 64;
  if (b < 1) b = 1;
  return static_cast<int>(b < kAuxBlocksMax ? b : kAuxBlocksMax);
}

// Per block partials: ws[b] = (P_0..P_{E-1}, c_0..c_{E-1}, W), fixed-order sums.
__global__ __launch_bounds__(kRouterWaves * kWave) void aux_partial_kernel(const float* __restrict__ logits,
                                                                            const float* __restrict__ token_weight,
                                                                            int T, int E, int k,
                                                                            float* __restrict__ ws) {
  __shared__ float part[kRouterWaves][2 * 1024 + 1];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int npl = (E + kWave - 1) / kWave;
  float P[kMaxPerLane], C[kMaxPerLane];
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) P[j] = C[j] = 0.0f;
  float W = 0.0f;
  const int waves_total = gridDim.x * kRouterWaves;
  for (int t = blockIdx.x * kRouterWaves + wave; t < T; t += waves_total) {
    float v[kMaxPerLane];
    load_row(logits + static_cast<int64_t>(t) * E, E, v, npl);
    SoftmaxStats st = softmax_stats(v, npl);
    int sel[kMaxTopK];
    float sl[kMaxTopK];
    select_topk(v, npl, E, k, sel, sl);
    const float w = token_weight ? token_weight[t] : 1.0f;
    W += w;
    const float inv_sum = 1.0f / st.sum;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      int e = lane + j * kWave;
      if (j < npl && e < E) {
        P[j] += w * (expf(v[j] - st.max) * inv_sum);
        float cnt = 0.0f;
#pragma unroll
        for (int r = 0; r < kMaxTopK; ++r)
          if (r < k && sel[r] == e) cnt += 1.0f;
        C[j] += w * cnt;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    int e = lane + j * kWave;
    if (j < npl && e < E) {
      part[wave][e] = P[j];
      part[wave][E + e] = C[j];
    }
  }
  if (lane == 0) part[wave][2 * E] = W;
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * E + 1; i += blockDim.x) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kRouterWaves; ++w) s += part[w][i];
    ws[static_cast<int64_t>(blockIdx.x) * (2 * E + 1) + i] = s;
  }
}

// Reduces the partials in block order; writes stats = (c_0..c_{E-1}, W), aux.
__global__ __launch_bounds__(1024) void aux_finalize_kernel(const float* __restrict__ ws, int nblk, int E,
                                                             float* __restrict__ stats, float* __restrict__ aux) {
  __shared__ float terms[1024];
  __shared__ float Wsh;
  const int tid = threadIdx.x;
  if (tid == 0) {
    float W = 0.0f;
    for (int b = 0; b < nblk; ++b) W += ws[static_cast<int64_t>(b) * (2 * E + 1) + 2 * E];
    Wsh = W;
    stats[E] = W;
  }
  __syncthreads();
  const float W = Wsh;
  for (int e = tid; e < 1024; e += blockDim.x) {
    float term = 0.0f;
    if (e < E) {
      float P = 0.0f, C = 0.0f;
      for (int b = 0; b < nblk; ++b) {
        P += ws[static_cast<int64_t>(b) * (2 * E + 1) + e];
        C += ws[static_cast<int64_t>(b) * (2 * E + 1) + E + e];
      }
      stats[e] = C;
      term = (C / W) * (P / W);
    }
    terms[e] = term;
  }
  __syncthreads();
  // Fixed-shape tree over 1024 terms.
  for (int s = 512; s >= 1; s >>= 1) {
    if (tid < s) terms[tid] += terms[tid + s];
    __syncthreads();
  }
  if (tid == 0) aux[0] = static_cast<float>(E) * terms[0];
}

__global__ __launch_bounds__(kRouterWaves * kWave) void aux_bwd_kernel(const float* __restrict__ logits,
                                                                        const float* __restrict__ token_weight,
                                                                        const float* __restrict__ stats,
                                                                        const float* __restrict__ d_aux, int T, int E,
                                                                        float* __restrict__ d_logits, int accumulate) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const int npl = (E + kWave - 1) / kWave;
  float v[kMaxPerLane];
  load_row(logits + static_cast<int64_t>(t) * E, E, v, npl);
  SoftmaxStats st = softmax_stats(v, npl);
  const float inv_sum = 1.0f / st.sum;
  const float W = stats[E];
  const float w = token_weight ? token_weight[t] : 1.0f;
  const float scale = d_aux[0] * static_cast<float>(E) * w / (W * W);
  float p[kMaxPerLane], g[kMaxPerLane];
  float dot = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    int e = lane + j * kWave;
    p[j] = 0.0f;
    g[j] = 0.0f;
    if (j < npl && e < E) {
      p[j] = expf(v[j] - st.max) * inv_sum;
      g[j] = scale * stats[e];
      dot += p[j] * g[j];
    }
  }
  dot = wave_sum(dot);
  float* drow = d_logits + static_cast<int64_t>(t) * E;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    int e = lane + j * kWave;
    if (j < npl && e < E) {
      float d = p[j] * (g[j] - dot);
      drow[e] = accumulate ? drow[e] + d : d;
    }
  }
}

}  // namespace moe

using namespace moe;

namespace {
int check_router(int64_t T, int64_t E, int64_t k) {
  MOE_REQUIRE(T >= 0 && T < (1ll << 31), MOE_ERR_INVALID, "router: bad token count %lld", (long long)T);
  MOE_REQUIRE(E >= 1 && E <= kMaxPerLane * kWave, MOE_ERR_UNSUPPORTED, "router: E=%lld outside [1,%d]", (long long)E,
              kMaxPerLane * kWave);
  MOE_REQUIRE(k >= 1 && k <= kMaxTopK && k <= E, MOE_ERR_UNSUPPORTED, "router: top_k=%lld outside [1,min(E,%d)]",
              (long long)k, kMaxTopK);
  return MOE_OK;
}
}  // namespace

extern "C" int moe_router_topk_fwd(const float* logits, float* scores, int64_t* indices, int64_t T, int64_t E,
                                   int64_t k, int norm_topk_prob, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  MOE_REQUIRE(logits && scores && indices, MOE_ERR_INVALID, "router topk: null pointer");
  if (T == 0) return MOE_OK;
  int blocks = static_cast<int>((T + kRouterWaves - 1) / kRouterWaves);
  hipLaunchKernelGGL(router_topk_fwd_kernel, dim3(blocks), dim3(kRouterWaves * kWave), 0, as_stream(stream), logits,
                     scores, indices, static_cast<int>(T), static_cast<int>(E), static_cast<int>(k),
                     norm_topk_prob ? 1 : 0);
  return launch_status("moe_router_topk_fwd");
}

extern "C" int moe_router_topk_bwd(const float* logits, const int64_t* indices, const float* d_scores, int64_t T,
                                   int64_t E, int64_t k, int norm_topk_prob, float* d_logits, int accumulate,
                                   void* d_logits_bf16, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  MOE_REQUIRE(logits && indices && d_scores && d_logits, MOE_ERR_INVALID, "router topk bwd: null pointer");
  if (T == 0) return MOE_OK;
  int blocks = static_cast<int>((T + kRouterWaves - 1) / kRouterWaves);
  hipLaunchKernelGGL(router_topk_bwd_kernel, dim3(blocks), dim3(kRouterWaves * kWave), 0, as_stream(stream), logits,
                     indices, d_scores, static_cast<int>(T), static_cast<int>(E), static_cast<int>(k),
                     norm_topk_prob ? 1 : 0, d_logits, accumulate ? 1 : 0, static_cast<bf16_t*>(d_logits_bf16));
  return launch_status("moe_router_topk_bwd");
}

extern "C" size_t moe_aux_loss_workspace_bytes(int64_t T, int64_t E) {
  if (T < 0 || E < 1) return 0;
  return static_cast<size_t>(aux_blocks(T)) * static_cast<size_t>(2 * E + 1) * sizeof(float);
}

extern "C" int moe_aux_loss_fwd(const float* logits, const float* token_weight, int64_t T, int64_t E, int64_t k,
                                float* aux, float* stats, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  MOE_REQUIRE(logits && aux && stats && workspace, MOE_ERR_INVALID, "aux loss: null pointer");
  MOE_REQUIRE(T >= 1, MOE_ERR_INVALID, "aux loss: needs at least one token");
  MOE_REQUIRE(workspace_bytes >= moe_aux_loss_workspace_bytes(T, E), MOE_ERR_WORKSPACE,
              "aux loss: workspace %zu < %zu bytes", workspace_bytes, moe_aux_loss_workspace_bytes(T, E));
  const int nblk = aux_blocks(T);
  float* ws = static_cast<float*>(workspace);
  hipLaunchKernelGGL(aux_partial_kernel, dim3(nblk), dim3(kRouterWaves * kWave), 0, as_stream(stream), logits,
                     token_weight, static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), ws);
  rc = launch_status("moe_aux_loss_fwd(partial)");
  if (rc) return rc;
  hipLaunchKernelGGL(aux_finalize_kernel, dim3(1), dim3(1024), 0, as_stream(stream), ws, nblk, static_cast<int>(E),
                     stats, aux);
  return launch_status("moe_aux_loss_fwd(finalize)");
}

extern "C" int moe_aux_loss_bwd(const float* logits, const float* token_weight, const float* stats, const float* d_aux,
                                int64_t T, int64_t E, float* d_logits, int accumulate, void* stream) {
  int rc = check_router(T, E, 1);
  if (rc) return rc;
  MOE_REQUIRE(logits && stats && d_aux && d_logits, MOE_ERR_INVALID, "aux loss bwd: null pointer");
  if (T == 0) return MOE_OK;
  int blocks = static_cast<int>((T + kRouterWaves - 1) / kRouterWaves);
  hipLaunchKernelGGL(aux_bwd_kernel, dim3(blocks), dim3(kRouterWaves * kWave), 0, as_stream(stream), logits,
                     token_weight, stats, d_aux, static_cast<int>(T), static_cast<int>(E), d_logits,
                     accumulate ? 1 : 0);
  return launch_status("moe_aux_loss_bwd");
}
