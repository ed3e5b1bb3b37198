// Weighted combine of expert rows back into token order, and its backward.
//
// Gather form, one 64-lane wave per token, 16 bytes (8 bf16) per lane per
// step: the k expert rows of a token are read, scaled and summed in fp32 and
// written once.  No atomics, so the result is deterministic; the backward
// reads each token's output gradient once and produces both the row gradients
// and the routing-score gradients (a wave dot product per routed slot); its
// fused form then runs the router's top-k backward on those gradients.
//
// Reference: TF/integrations/moe.py:461-478 (weight, mask, inverse permute,
// sum over k in fp32) and parallel/parallel/engine/model_parallel/
// token_dispatch.py:160-174 (index_add combine, unweighted).
#include "common.h"
#include "router_token.h"

namespace moe {

constexpr int kCombThreads = 256;
constexpr int kCombWaves = kCombThreads / kWave;

__device__ __forceinline__ void unpack8(const uint4& v, float (&f)[8]) {
  f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x);
  f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
  f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z);
  f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  uint4 o;
  o.x = pack_bf16x2(f[0], f[1]);
  o.y = pack_bf16x2(f[2], f[3]);
  o.z = pack_bf16x2(f[4], f[5]);
  o.w = pack_bf16x2(f[6], f[7]);
  return o;
}

template <int KT>
__global__ __launch_bounds__(kCombThreads) void combine_fwd_kernel(const bf16_t* __restrict__ y,
                                                                    const int32_t* __restrict__ pos_of_slot,
                                                                    const int32_t* __restrict__ n_valid_ptr,
                                                                    const float* __restrict__ scores, int T, int H,
                                                                    int k, bf16_t* __restrict__ out) {
  constexpr int KM = Slots<KT>::KM;
  const int lane = threadIdx.x & (kWave - 1);
  const int n_valid = *n_valid_ptr;
  const int nchunk = H / 8;
  for (int t = blockIdx.x * kCombWaves + (threadIdx.x >> 6); t < T; t += gridDim.x * kCombWaves) {
    Slots<KT> sl;
    sl.load(pos_of_slot, scores, t, k, n_valid);
    for (int c = lane; c < nchunk; c += kWave) {
      // Every live slot's row load is issued before any is used; rows are
      // added in slot order.
      uint4 v[KM];
#pragma unroll
      for (int j = 0; j < KM; ++j)
        if (KT || j < k) v[j] = reinterpret_cast<const uint4*>(y + static_cast<int64_t>(sl.pos[j]) * H)[c];
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        if (sl.ok[j]) {
          float f[8];
          unpack8(v[j], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += f[e] * sl.w[j];
        }
      }
      reinterpret_cast<uint4*>(out + static_cast<int64_t>(t) * H)[c] = pack8(acc);
    }
  }
}

// One token's combine backward: d_y[slot] = s_slot * d_out[t] for each of
// its k slots (zero rows for slots without a row) and, with_scores, the
// routing weights' gradient ds[j] = <y[slot j], d_out[t]> (the same value in
// every lane).
template <int KT>
__device__ __forceinline__ void combine_bwd_token(const bf16_t* __restrict__ d_out, const bf16_t* __restrict__ y,
                                                  const int32_t* __restrict__ pos_of_slot, int n_valid,
                                                  const float* __restrict__ scores, int64_t t, int H, int k,
                                                  bf16_t* __restrict__ d_y, bool with_scores,
                                                  float (&ds)[Slots<KT>::KM]) {
  constexpr int KM = Slots<KT>::KM;
  const int lane = threadIdx.x & (kWave - 1);
  const int nchunk = H / 8;
  Slots<KT> sl;
  sl.load(pos_of_slot, scores, t, k, n_valid);
  // Slots without a row still get their (zero) gradient row written.
  int dst_row[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    const bool live = KT ? true : j < k;
    dst_row[j] = __builtin_amdgcn_readfirstlane(live ? pos_of_slot[t * k + j] : 0);
  }
  float dot[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) dot[j] = 0.0f;
  for (int c = lane; c < nchunk; c += kWave) {
    float g[8];
    unpack8(reinterpret_cast<const uint4*>(d_out + t * H)[c], g);
    uint4 v[KM];
    if (with_scores) {
#pragma unroll
      for (int j = 0; j < KM; ++j)
        if (KT || j < k)  // the backward's last read of the expert outputs
          v[j] = ntload16(reinterpret_cast<const uint4*>(y + static_cast<int64_t>(sl.pos[j]) * H) + c);
    }
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      if (KT || j < k) {
        uint4* dst = reinterpret_cast<uint4*>(d_y + static_cast<int64_t>(dst_row[j]) * H) + c;
        if (sl.ok[j]) {
          if (with_scores) {
            float f[8];
            unpack8(v[j], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) dot[j] += f[e] * g[e];
          }
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = g[e] * sl.w[j];
          *dst = pack8(o);
        } else {
          *dst = make_uint4(0, 0, 0, 0);
        }
      }
    }
  }
  if (with_scores) {
#pragma unroll
    for (int j = 0; j < KM; ++j) ds[j] = (KT || j < k) ? wave_sum(dot[j]) : 0.0f;
  }
}

template <int KT>
__global__ __launch_bounds__(kCombThreads) void combine_bwd_kernel(const bf16_t* __restrict__ d_out,
                                                                    const bf16_t* __restrict__ y,
                                                                    const int32_t* __restrict__ pos_of_slot,
                                                                    const int32_t* __restrict__ n_valid_ptr,
                                                                    const float* __restrict__ scores, int T, int H,
                                                                    int k, bf16_t* __restrict__ d_y,
                                                                    float* __restrict__ d_scores) {
  constexpr int KM = Slots<KT>::KM;
  const int lane = threadIdx.x & (kWave - 1);
  const int n_valid = *n_valid_ptr;
  for (int t = blockIdx.x * kCombWaves + (threadIdx.x >> 6); t < T; t += gridDim.x * kCombWaves) {
    float ds[KM];
    combine_bwd_token<KT>(d_out, y, pos_of_slot, n_valid, scores, t, H, k, d_y, d_scores != nullptr, ds);
    if (d_scores && lane == 0) {
#pragma unroll
      for (int j = 0; j < KM; ++j)
        if (KT || j < k) d_scores[static_cast<int64_t>(t) * k + j] = ds[j];
    }
  }
}

// The combine backward of a token followed by the router's top-k backward
// of the same token (the one-op block's backward): the routing weights'
// gradient goes from the combine's dot products straight into the top-k
// backward (and to d_scores when asked for), and the token's logits and
// selection are loaded before its rows are streamed.  The results are the
// bits of combine_bwd_kernel followed by router_topk_bwd_kernel on its
// d_scores.
template <int KT, int NPL>
__global__ __launch_bounds__(kCombThreads) void combine_router_bwd_kernel(
    const bf16_t* __restrict__ d_out, const bf16_t* __restrict__ y, const int32_t* __restrict__ pos_of_slot,
    const int32_t* __restrict__ n_valid_ptr, const float* __restrict__ scores, int T, int H, int k,
    bf16_t* __restrict__ d_y, float* __restrict__ d_scores, const float* __restrict__ logits,
    const int64_t* __restrict__ indices, const float* d_add, int E, int norm, const float* __restrict__ token_weight,
    const float* __restrict__ aux_stats, const float* __restrict__ d_aux, int bf16_terms,
    bf16_t* __restrict__ d_logits_bf16) {
  using Row = TopkBwdRow<kWave, NPL, KT>;
  static_assert(Row::KM == Slots<KT>::KM, "one score gradient per slot");
  const int lane = threadIdx.x & (kWave - 1);
  const int n_valid = *n_valid_ptr;
  for (int tw = blockIdx.x * kCombWaves + (threadIdx.x >> 6); tw < T; tw += gridDim.x * kCombWaves) {
    const int t = __builtin_amdgcn_readfirstlane(tw);  // the wave's token: its routes and scalars load once
    Row row;
    topk_bwd_load(row, logits, indices, d_add, t, E, k, token_weight, aux_stats, d_aux);
    float ds[Row::KM];
    combine_bwd_token<KT>(d_out, y, pos_of_slot, n_valid, scores, t, H, k, d_y, true, ds);
    if (d_scores && lane == 0) {
#pragma unroll
      for (int j = 0; j < Row::KM; ++j)
        if (KT || j < k) d_scores[static_cast<int64_t>(t) * k + j] = ds[j];
    }
    topk_bwd_finish(row, ds, logits, t, E, k, norm, d_add != nullptr, aux_stats != nullptr, nullptr, d_logits_bf16,
                    bf16_terms);
  }
}

int token_grid(int64_t T) {
  int64_t b = (T + kCombWaves - 1) / kCombWaves;
  if (b > 8192) b = 8192;
  return static_cast<int>(b < 1 ? 1 : b);
}

int check_combine(const void* rows, const int32_t* pos_of_slot, const int32_t* offsets, int64_t nb, int64_t T,
                  int64_t H, int64_t k, const void* out) {
  MOE_REQUIRE(T >= 0 && T < (1ll << 31) && k >= 1 && k <= kMaxSlots && H > 0 && H % 8 == 0, MOE_ERR_INVALID,
              "combine: bad sizes T=%lld H=%lld k=%lld (H %% 8 == 0, 1 <= k <= %d)", (long long)T, (long long)H,
              (long long)k, kMaxSlots);
  MOE_REQUIRE(nb >= 1, MOE_ERR_INVALID, "combine: num_buckets must be >= 1");
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(rows && pos_of_slot && offsets && out, MOE_ERR_INVALID, "combine: null pointer");
  MOE_REQUIRE(aligned16(rows) && aligned16(out), MOE_ERR_INVALID, "combine: buffers must be 16-byte aligned");
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_combine_fwd(const void* y, const int32_t* pos_of_slot, const int32_t* offsets,
                               int64_t num_buckets, const float* scores, int64_t T, int64_t H, int64_t k, void* out,
                               void* stream) {
  int rc = check_combine(y, pos_of_slot, offsets, num_buckets, T, H, k, out);
  if (rc || T == 0) return rc;
  MOE_DISPATCH_K(k, combine_fwd_kernel, dim3(token_grid(T)), dim3(kCombThreads), 0, as_stream(stream),
                     static_cast<const bf16_t*>(y), pos_of_slot, offsets + (num_buckets - 1), scores,
                     static_cast<int>(T), static_cast<int>(H), static_cast<int>(k), static_cast<bf16_t*>(out));
  return launch_status("moe_combine_fwd");
}

extern "C" int moe_combine_bwd(const void* d_out, const void* y, const int32_t* pos_of_slot, const int32_t* offsets,
                               int64_t num_buckets, const float* scores, int64_t T, int64_t H, int64_t k, void* d_y,
                               float* d_scores, void* stream) {
  int rc = check_combine(d_out, pos_of_slot, offsets, num_buckets, T, H, k, d_y);
  if (rc || T == 0) return rc;
  MOE_REQUIRE(!d_scores || (y && aligned16(y)), MOE_ERR_INVALID, "combine bwd: d_scores needs y");
  MOE_DISPATCH_K(k, combine_bwd_kernel, dim3(token_grid(T)), dim3(kCombThreads), 0, as_stream(stream),
                     static_cast<const bf16_t*>(d_out), static_cast<const bf16_t*>(y), pos_of_slot,
                     offsets + (num_buckets - 1), scores, static_cast<int>(T), static_cast<int>(H),
                     static_cast<int>(k), static_cast<bf16_t*>(d_y), d_scores);
  return launch_status("moe_combine_bwd");
}

extern "C" int moe_combine_router_bwd(const void* d_out, const void* y, const int32_t* pos_of_slot,
                                      const int32_t* offsets, int64_t num_buckets, const float* scores, int64_t T,
                                      int64_t H, int64_t k, void* d_y, float* d_scores, const float* logits,
                                      const int64_t* indices, const float* d_logits, const float* token_weight,
                                      const float* stats, const float* d_aux, int64_t E, int norm_topk_prob,
                                      int bf16_terms, void* d_logits_bf16, void* stream) {
  int rc = check_combine(d_out, pos_of_slot, offsets, num_buckets, T, H, k, d_y);
  if (rc) return rc;
  MOE_REQUIRE(E >= 1 && E <= kMaxPerLane * kWave, MOE_ERR_UNSUPPORTED, "combine router bwd: E=%lld outside [1,%d]",
              (long long)E, kMaxPerLane * kWave);
  MOE_REQUIRE(k <= kMaxTopK && k <= E, MOE_ERR_UNSUPPORTED, "combine router bwd: top_k=%lld outside [1,min(E,%d)]",
              (long long)k, kMaxTopK);
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(y && aligned16(y) && logits && indices && d_logits_bf16, MOE_ERR_INVALID,
              "combine router bwd: null or misaligned pointer");
  MOE_REQUIRE(!stats == !d_aux, MOE_ERR_INVALID, "combine router bwd: stats and d_aux go together");
  with_npl_k<true>(E, k, [&](auto L, auto N, auto K) {
    static_assert(decltype(L)::value == kWave, "one wave per token");
    hipLaunchKernelGGL((combine_router_bwd_kernel<decltype(K)::value, decltype(N)::value>), dim3(token_grid(T)),
                       dim3(kCombThreads), 0, as_stream(stream), static_cast<const bf16_t*>(d_out),
                       static_cast<const bf16_t*>(y), pos_of_slot, offsets + (num_buckets - 1), scores,
                       static_cast<int>(T), static_cast<int>(H), static_cast<int>(k), static_cast<bf16_t*>(d_y),
                       d_scores, logits, indices, d_logits, static_cast<int>(E), norm_topk_prob ? 1 : 0,
                       token_weight, stats, d_aux, bf16_terms ? 1 : 0, static_cast<bf16_t*>(d_logits_bf16));
  });
  return launch_status("moe_combine_router_bwd");
}
