// RMSNorm of the MoE block's input (the decoder layer's
// post_attention_layernorm), forward and backward, on gfx950.
//
// Reference: Qwen3MoeRMSNorm.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299,
// applied before the MoE block at :345 (the router and the experts both read
// its output):
//   hs = h.float() * rsqrt(mean(h.float()^2, -1) + eps);   x = weight * hs.to(bf16)
// so x = bf16(weight * bf16(hs)) with fp32 statistics.  Its autograd gives
//   g   = bf16(dx (+ dx2))                 (autograd adds the two consumers' bf16 grads)
//   dhs = bf16(g * weight)                 (bf16 product, then cast to fp32 by .to())
//   dh  = bf16(r dhs - (r^3 / H) h sum_j(dhs_j h_j)),  r = rsqrt(mean(h^2) + eps)
//   dweight = bf16(sum_t bf16(g * bf16(hs)))
//
// One 64-lane wave per row, 8 bf16 per lane per chunk, the row in registers
// (H <= 64 * 8 * kNormMaxChunks).  The weight gradient is a column sum over
// the rows: per-block partials (each block's 4 rows, wave order), then row
// groups, then the groups in order; every sum has a fixed order.
#include "common.h"

namespace moe {

constexpr int kNormWaves = 4;       // rows per block
constexpr int kNormMaxChunks = 8;   // 16-byte chunks per lane: H <= 4096
constexpr int kNormGroups = 16;     // row groups of the weight-gradient reduction

__device__ __forceinline__ void unpack8f(const uint4& v, float (&f)[8]) {
  f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x);
  f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
  f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z);
  f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
}
__device__ __forceinline__ uint4 pack8f(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}
__device__ __forceinline__ float round_bf16f(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__global__ __launch_bounds__(kNormWaves * kWave) void rmsnorm_fwd_kernel(const bf16_t* __restrict__ h,
                                                                          const bf16_t* __restrict__ gamma, int T,
                                                                          int H, float eps, bf16_t* __restrict__ x,
                                                                          float* __restrict__ rstd) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * kNormWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nchunk = H / 8;
  const uint4* row = reinterpret_cast<const uint4*>(h + static_cast<int64_t>(t) * H);
  uint4 v[kNormMaxChunks];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    const int c = lane + i * kWave;
    if (c < nchunk) {
      v[i] = row[c];
      float f[8];
      unpack8f(v[i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(H) + eps);
  if (lane == 0) rstd[t] = r;
  uint4* out = reinterpret_cast<uint4*>(x + static_cast<int64_t>(t) * H);
  const uint4* gw = reinterpret_cast<const uint4*>(gamma);
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    const int c = lane + i * kWave;
    if (c < nchunk) {
      float f[8], g[8];
      unpack8f(v[i], f);
      unpack8f(gw[c], g);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = g[e] * round_bf16f(f[e] * r);
      out[c] = pack8f(f);
    }
  }
}

// dh per row, and per-block partial column sums of bf16(g * bf16(hs)) into
// partials[block][H] (the block's rows added in wave order).
__global__ __launch_bounds__(kNormWaves * kWave) void rmsnorm_bwd_kernel(
    const bf16_t* __restrict__ dx, const bf16_t* __restrict__ dx2, const bf16_t* __restrict__ h,
    const bf16_t* __restrict__ gamma, const float* __restrict__ rstd, int T, int H, bf16_t* __restrict__ dh,
    float* __restrict__ partials) {
  __shared__ float part[kNormWaves][kNormMaxChunks * 8 * kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int t = blockIdx.x * kNormWaves + wave;
  const int nchunk = H / 8;
  const bool live = t < T;
  float dg[kNormMaxChunks][8];  // this row's contribution to the weight gradient
  if (live) {
    const int64_t base = static_cast<int64_t>(t) * H;
    const uint4* hr = reinterpret_cast<const uint4*>(h + base);
    const uint4* gr = reinterpret_cast<const uint4*>(dx + base);
    const uint4* gr2 = dx2 ? reinterpret_cast<const uint4*>(dx2 + base) : nullptr;
    const uint4* gw = reinterpret_cast<const uint4*>(gamma);
    const float r = rstd[t];
    float hv[kNormMaxChunks][8], dhs[kNormMaxChunks][8];
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) {
      const int c = lane + i * kWave;
#pragma unroll
      for (int e = 0; e < 8; ++e) dg[i][e] = hv[i][e] = dhs[i][e] = 0.0f;
      if (c < nchunk) {
        float g[8], g2[8], w[8];
        unpack8f(hr[c], hv[i]);
        unpack8f(gr[c], g);
        unpack8f(gw[c], w);
        if (gr2) {
          unpack8f(gr2[c], g2);
#pragma unroll
          for (int e = 0; e < 8; ++e) g[e] = round_bf16f(g[e] + g2[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dhs[i][e] = round_bf16f(g[e] * w[e]);
          dot += dhs[i][e] * hv[i][e];
          dg[i][e] = round_bf16f(g[e] * round_bf16f(hv[i][e] * r));
        }
      }
    }
    dot = wave_sum(dot);
    const float k3 = r * r * r / static_cast<float>(H);
    uint4* out = reinterpret_cast<uint4*>(dh + base);
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) {
      const int c = lane + i * kWave;
      if (c < nchunk) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = r * dhs[i][e] - k3 * hv[i][e] * dot;
        out[c] = pack8f(o);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) dg[i][e] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) part[wave][(i * kWave + lane) * 8 + e] = dg[i][e];
  __syncthreads();
  float* prow = partials + static_cast<int64_t>(blockIdx.x) * H;
  for (int j = threadIdx.x; j < H; j += blockDim.x) {
    // column j lives at chunk j/8 = i*64 + lane, element j%8
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kNormWaves; ++w) s += part[w][j];
    prow[j] = s;
  }
}

// sums[g][j] = sum over the partial rows of group g (rows [g*per, (g+1)*per)),
// wave w adding rows w, w+4, ... and the waves combined in order.
__global__ __launch_bounds__(256) void colsum_groups_kernel(const float* __restrict__ partials, int nrows, int n,
                                                            float* __restrict__ sums) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  const int g = blockIdx.y;
  const int per = (nrows + kNormGroups - 1) / kNormGroups;
  const int r0 = g * per, r1 = min(nrows, r0 + per);
  float acc = 0.0f;
  if (col < n) {
#pragma unroll 8
    for (int r = r0 + wave; r < r1; r += 4) acc += partials[static_cast<int64_t>(r) * n + col];
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && col < n)
    sums[static_cast<int64_t>(g) * n + col] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
}

__global__ __launch_bounds__(256) void colsum_finalize_bf16_kernel(const float* __restrict__ sums, int n,
                                                                   bf16_t* __restrict__ out) {
  const int col = blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= n) return;
  float q[kNormGroups];
#pragma unroll
  for (int g = 0; g < kNormGroups; ++g) q[g] = sums[static_cast<int64_t>(g) * n + col];
  float s = 0.0f;
#pragma unroll
  for (int g = 0; g < kNormGroups; ++g) s += q[g];
  out[col] = f32_to_bf16(s);
}

}  // namespace moe

using namespace moe;

namespace {
int check_norm(const void* a, const void* gamma, int64_t T, int64_t H) {
  MOE_REQUIRE(a && gamma, MOE_ERR_INVALID, "rmsnorm: null pointer");
  MOE_REQUIRE(T >= 0 && T < (1ll << 31), MOE_ERR_INVALID, "rmsnorm: bad row count %lld", (long long)T);
  MOE_REQUIRE(H > 0 && H % 8 == 0 && H <= 64 * 8 * kNormMaxChunks, MOE_ERR_UNSUPPORTED,
              "rmsnorm: H=%lld must be a multiple of 8 and at most %d", (long long)H, 64 * 8 * kNormMaxChunks);
  MOE_REQUIRE(aligned16(a) && aligned16(gamma), MOE_ERR_INVALID, "rmsnorm: operands must be 16-byte aligned");
  return MOE_OK;
}
int64_t norm_blocks(int64_t T) { return (T + kNormWaves - 1) / kNormWaves; }
}  // namespace

extern "C" int moe_rmsnorm_fwd(const void* h, const void* gamma, int64_t T, int64_t H, float eps, void* x,
                               float* rstd, void* stream) {
  int rc = check_norm(h, gamma, T, H);
  if (rc) return rc;
  MOE_REQUIRE(x && rstd && aligned16(x), MOE_ERR_INVALID, "rmsnorm fwd: bad output pointer");
  MOE_REQUIRE(eps >= 0.0f, MOE_ERR_INVALID, "rmsnorm fwd: eps must be non-negative");
  if (T == 0) return MOE_OK;
  hipLaunchKernelGGL(rmsnorm_fwd_kernel, dim3(static_cast<unsigned>(norm_blocks(T))), dim3(kNormWaves * kWave), 0,
                     as_stream(stream), static_cast<const bf16_t*>(h), static_cast<const bf16_t*>(gamma),
                     static_cast<int>(T), static_cast<int>(H), eps, static_cast<bf16_t*>(x), rstd);
  return launch_status("moe_rmsnorm_fwd");
}

extern "C" size_t moe_rmsnorm_bwd_workspace_bytes(int64_t T, int64_t H) {
  if (T < 0 || H < 1) return 0;
  return static_cast<size_t>(norm_blocks(T) + kNormGroups) * static_cast<size_t>(H) * sizeof(float);
}

extern "C" int moe_rmsnorm_bwd(const void* dx, const void* dx2, const void* h, const void* gamma, const float* rstd,
                               int64_t T, int64_t H, void* dh, void* dgamma, void* workspace, size_t workspace_bytes,
                               void* stream) {
  int rc = check_norm(h, gamma, T, H);
  if (rc) return rc;
  MOE_REQUIRE(dx && rstd && dh && dgamma && aligned16(dx) && aligned16(dh) && (!dx2 || aligned16(dx2)),
              MOE_ERR_INVALID, "rmsnorm bwd: bad pointer");
  const size_t need = moe_rmsnorm_bwd_workspace_bytes(T, H);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE, "rmsnorm bwd: workspace %zu < %zu bytes",
              workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  const int nblk = static_cast<int>(norm_blocks(T));
  float* partials = static_cast<float*>(workspace);
  float* sums = partials + static_cast<int64_t>(nblk) * H;
  if (T > 0) {
    hipLaunchKernelGGL(rmsnorm_bwd_kernel, dim3(nblk), dim3(kNormWaves * kWave), 0, st,
                       static_cast<const bf16_t*>(dx), static_cast<const bf16_t*>(dx2),
                       static_cast<const bf16_t*>(h), static_cast<const bf16_t*>(gamma), rstd, static_cast<int>(T),
                       static_cast<int>(H), static_cast<bf16_t*>(dh), partials);
    rc = launch_status("moe_rmsnorm_bwd(rows)");
    if (rc) return rc;
  }
  const int n = static_cast<int>(H);
  hipLaunchKernelGGL(colsum_groups_kernel, dim3((n + 63) / 64, kNormGroups), dim3(256), 0, st, partials, nblk, n,
                     sums);
  rc = launch_status("moe_rmsnorm_bwd(groups)");
  if (rc) return rc;
  hipLaunchKernelGGL(colsum_finalize_bf16_kernel, dim3((n + 255) / 256), dim3(256), 0, st, sums, n,
                     static_cast<bf16_t*>(dgamma));
  return launch_status("moe_rmsnorm_bwd(finalize)");
}
