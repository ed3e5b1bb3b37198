// The fp32 expert path.
//
// The reference's grouped experts run in the modules' dtype, fp32 included
// (TF/integrations/moe.py:377-478: F.grouped_mm over the permuted rows,
// act_fn(gate) * up, the weighted sum over the k routes).  These kernels run
// that path on gfx950 with fp32 operands and fp32 arithmetic throughout:
//   - one grouped GEMM, C(i, j) (+)= sum_r A(i, r) B(r, j) with arbitrary
//     strides, on v_mfma_f32_32x32x2_f32 (one 32x32 output tile per wave),
//     grouped over the output rows (the projections and their input
//     gradients: rows of group g use weight g) or over the reduction rows
//     (the weight gradients: group g's rows give weight g's gradient);
//   - one wave per row for SwiGLU, its backward, the weighted combine, its
//     backward and the permute backward.
// It serves fp32 modules (the C1 configuration); the bf16 path is the tuned
// one.  The row permutation itself is moe_permute_fwd over the rows' bytes.
#include <algorithm>

#include "common.h"

namespace moe {
namespace {

constexpr int kF32Waves = 4;  // waves (32x32 tiles) per block

struct F32Gemm {
  const float* A;
  const float* B;
  float* C;
  const int32_t* offs;
  int G, mode, M, N, K;  // mode 0: groups over i (M rows in all), 1: groups over r (K rows in all)
  int64_t sAi, sAr, sBr, sBj, sCi, sCj, sBg, sCg;
  int accumulate;
};

// Group g's rows [lo, hi) from the inclusive offsets, clamped to [0, n).
__device__ __forceinline__ void f32_group_rows(const int32_t* offs, int g, int n, int& lo, int& hi) {
  lo = g ? min(max(offs[g - 1], 0), n) : 0;
  hi = min(max(offs[g], lo), n);
}

// One wave per 32x32 tile of C.  Lane l of an MFMA step supplies A(i0 + l % 32,
// r + l / 32) and B(r + l / 32, j0 + l % 32), and holds D rows
// 8 (q / 4) + 4 (l / 32) + q % 4 (q = 0..15) of column j0 + l % 32.
__global__ __launch_bounds__(kF32Waves * kWave) void f32_grouped_gemm_kernel(const F32Gemm p, int tiles_j,
                                                                            int64_t ntiles) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * kF32Waves + (threadIdx.x >> 6);
  if (tile >= ntiles) return;
  const int tj = static_cast<int>(tile % tiles_j);
  int64_t rest = tile / tiles_j;
  int g = 0, i_begin = 0, i_end = p.M, r_begin = 0, r_end = p.K, i0;
  if (p.mode == 0) {
    // the rest-th 32-row tile over the groups' row ranges
    int t = static_cast<int>(rest);
    g = -1;
    for (int gg = 0; gg < p.G; ++gg) {
      int lo, hi;
      f32_group_rows(p.offs, gg, p.M, lo, hi);
      const int nt = (hi - lo + 31) / 32;
      if (t < nt) {
        g = gg;
        i_begin = lo;
        i_end = hi;
        break;
      }
      t -= nt;
    }
    if (g < 0) return;  // past the last tile (the grid is sized for the worst case)
    i0 = i_begin + 32 * t;
  } else {
    const int tiles_i = (p.M + 31) / 32;
    g = static_cast<int>(rest / tiles_i);
    i0 = 32 * static_cast<int>(rest % tiles_i);
    if (p.K > 0) f32_group_rows(p.offs, g, p.K, r_begin, r_end);  // no reduction rows: every group is empty
  }
  const int j0 = 32 * tj;
  const float* B = p.B + (p.mode == 0 ? static_cast<int64_t>(g) * p.sBg : 0);
  float* C = p.C + (p.mode == 1 ? static_cast<int64_t>(g) * p.sCg : 0);
  const int ia = i0 + (lane & 31), jb = j0 + (lane & 31), rl = lane >> 5;
  const bool ia_ok = ia < i_end, jb_ok = jb < p.N;
  f32x16_t acc;
#pragma unroll
  for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
  for (int r0 = r_begin; r0 < r_end; r0 += 16) {
    float a[8], b[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int r = r0 + 2 * u + rl;
      const bool r_ok = r < r_end;
      a[u] = (ia_ok && r_ok) ? p.A[static_cast<int64_t>(ia) * p.sAi + static_cast<int64_t>(r) * p.sAr] : 0.0f;
      b[u] = (jb_ok && r_ok) ? B[static_cast<int64_t>(r) * p.sBr + static_cast<int64_t>(jb) * p.sBj] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b[u], acc, 0, 0, 0);
  }
  if (!jb_ok) return;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int i = i0 + 8 * (q / 4) + 4 * (lane >> 5) + (q % 4);
    if (i < i_end) {
      float* c = C + static_cast<int64_t>(i) * p.sCi + static_cast<int64_t>(jb) * p.sCj;
      *c = p.accumulate ? *c + acc[q] : acc[q];
    }
  }
}

// act[r, c] = silu(pre[r, c]) * pre[r, I + c] for the rows below n_valid.
__global__ void f32_swiglu_fwd_kernel(const float* __restrict__ pre, float* __restrict__ act, int S, int I,
                                      const int32_t* __restrict__ n_valid_ptr) {
  const int n_valid = min(*n_valid_ptr, S);
  for (int r = blockIdx.x; r < n_valid; r += gridDim.x) {
    const float* row = pre + static_cast<int64_t>(r) * 2 * I;
    for (int c = threadIdx.x; c < I; c += blockDim.x) {
      const float gt = row[c];
      act[static_cast<int64_t>(r) * I + c] = gt / (1.0f + expf(-gt)) * row[I + c];
    }
  }
}

// d_pre[r] = (d_act * up * silu'(gate), d_act * silu(gate)) for the rows below n_valid.
__global__ void f32_swiglu_bwd_kernel(const float* __restrict__ d_act, const float* __restrict__ pre,
                                      float* __restrict__ d_pre, int S, int I,
                                      const int32_t* __restrict__ n_valid_ptr) {
  const int n_valid = min(*n_valid_ptr, S);
  for (int r = blockIdx.x; r < n_valid; r += gridDim.x) {
    const float* row = pre + static_cast<int64_t>(r) * 2 * I;
    float* drow = d_pre + static_cast<int64_t>(r) * 2 * I;
    for (int c = threadIdx.x; c < I; c += blockDim.x) {
      const float gt = row[c], up = row[I + c], da = d_act[static_cast<int64_t>(r) * I + c];
      const float s = 1.0f / (1.0f + expf(-gt));
      drow[c] = da * up * (s * (1.0f + gt * (1.0f - s)));
      drow[I + c] = da * gt * s;
    }
  }
}

// out[t] = sum_j w[t, j] y[pos(t, j)] over the token's slots below n_valid.
__global__ void f32_combine_fwd_kernel(const float* __restrict__ y, const int32_t* __restrict__ pos_of_slot,
                                       const int32_t* __restrict__ n_valid_ptr, const float* __restrict__ w, int T,
                                       int H, int k, float* __restrict__ out) {
  const int n_valid = *n_valid_ptr;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    for (int c = threadIdx.x; c < H; c += blockDim.x) {
      float acc = 0.0f;
      for (int j = 0; j < k; ++j) {
        const int p = pos_of_slot[static_cast<int64_t>(t) * k + j];
        if (p < n_valid) acc += w[static_cast<int64_t>(t) * k + j] * y[static_cast<int64_t>(p) * H + c];
      }
      out[static_cast<int64_t>(t) * H + c] = acc;
    }
  }
}

// d_y[pos(t, j)] = w[t, j] d_out[t] (zeros for sentinel slots); d_w[t, j] =
// <y[pos(t, j)], d_out[t]> (zero for sentinel slots).  One block per token.
__global__ void f32_combine_bwd_kernel(const float* __restrict__ d_out, const float* __restrict__ y,
                                       const int32_t* __restrict__ pos_of_slot,
                                       const int32_t* __restrict__ n_valid_ptr, const float* __restrict__ w, int T,
                                       int H, int k, float* __restrict__ d_y, float* __restrict__ d_w) {
  __shared__ float part[kMaxSlots][4];
  const int n_valid = *n_valid_ptr;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    float dot[kMaxSlots];
    for (int j = 0; j < kMaxSlots; ++j) dot[j] = 0.0f;
    for (int c = threadIdx.x; c < H; c += blockDim.x) {
      const float g = d_out[static_cast<int64_t>(t) * H + c];
      for (int j = 0; j < k; ++j) {
        const int p = pos_of_slot[static_cast<int64_t>(t) * k + j];
        const bool ok = p < n_valid;
        d_y[static_cast<int64_t>(p) * H + c] = ok ? w[static_cast<int64_t>(t) * k + j] * g : 0.0f;
        if (ok) dot[j] += y[static_cast<int64_t>(p) * H + c] * g;
      }
    }
    for (int j = 0; j < k; ++j) {
      const float s = wave_sum(dot[j]);
      if (lane == 0) part[j][wave] = s;
    }
    __syncthreads();
    if (threadIdx.x < k) {
      const int j = threadIdx.x;
      const int p = pos_of_slot[static_cast<int64_t>(t) * k + j];
      d_w[static_cast<int64_t>(t) * k + j] = p < n_valid ? ((part[j][0] + part[j][1]) + part[j][2]) + part[j][3] : 0.0f;
    }
    __syncthreads();
  }
}

// d_x[t] = sum_j d_xp[pos(t, j)] over the token's slots below n_valid, then
// + d_add[t] when given (the router's input gradient, added as autograd
// would add it to the experts' sum).
__global__ void f32_permute_bwd_kernel(const float* __restrict__ d_xp, const int32_t* __restrict__ pos_of_slot,
                                       const int32_t* __restrict__ n_valid_ptr, int T, int H, int k,
                                       const float* __restrict__ d_add, float* __restrict__ d_x) {
  const int n_valid = *n_valid_ptr;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    for (int c = threadIdx.x; c < H; c += blockDim.x) {
      float acc = 0.0f;
      for (int j = 0; j < k; ++j) {
        const int p = pos_of_slot[static_cast<int64_t>(t) * k + j];
        if (p < n_valid) acc += d_xp[static_cast<int64_t>(p) * H + c];
      }
      if (d_add) acc += d_add[static_cast<int64_t>(t) * H + c];
      d_x[static_cast<int64_t>(t) * H + c] = acc;
    }
  }
}

int rows_grid(int64_t rows) { return static_cast<int>(std::min<int64_t>(std::max<int64_t>(rows, 1), 65535)); }

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" int moe_f32_grouped_gemm(const float* A, const float* B, const int32_t* offs, int64_t G, int mode,
                                    int64_t M, int64_t N, int64_t K, int64_t sAi, int64_t sAr, int64_t sBr,
                                    int64_t sBj, int64_t sBg, float* C, int64_t sCi, int64_t sCj, int64_t sCg,
                                    int accumulate, void* stream) {
  MOE_REQUIRE(mode == 0 || mode == 1, MOE_ERR_INVALID, "f32 grouped gemm: mode must be 0 or 1");
  MOE_REQUIRE(G >= 1 && G <= 4096 && M >= 0 && N >= 0 && K >= 0 && M < (1ll << 31) && N < (1ll << 31) &&
                  K < (1ll << 31),
              MOE_ERR_INVALID, "f32 grouped gemm: bad sizes G=%lld M=%lld N=%lld K=%lld", (long long)G,
              (long long)M, (long long)N, (long long)K);
  if (N == 0 || M == 0) return MOE_OK;  // nothing to write: empty buffers may be NULL
  // A and B are read only when K > 0, offs always in mode 0 and only when K > 0 in mode 1
  MOE_REQUIRE(C && (K == 0 || (A && B)) && (offs || (mode == 1 && K == 0)), MOE_ERR_INVALID,
              "f32 grouped gemm: null pointer");
  F32Gemm p{A, B, C, offs, static_cast<int>(G), mode, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
            sAi, sAr, sBr, sBj, sCi, sCj, sBg, sCg, accumulate ? 1 : 0};
  const int tiles_j = static_cast<int>((N + 31) / 32);
  // mode 0: every group's rows in 32-row tiles, at most M / 32 + G of them
  const int64_t tiles_i = mode == 0 ? (M + 31) / 32 + G : G * ((M + 31) / 32);
  const int64_t ntiles = tiles_i * tiles_j;
  const int64_t blocks = (ntiles + kF32Waves - 1) / kF32Waves;
  MOE_REQUIRE(blocks < (1ll << 31), MOE_ERR_UNSUPPORTED, "f32 grouped gemm: too many tiles");
  hipLaunchKernelGGL(f32_grouped_gemm_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kF32Waves * kWave), 0,
                     as_stream(stream), p, tiles_j, ntiles);
  return launch_status("moe_f32_grouped_gemm");
}

extern "C" int moe_f32_swiglu_fwd(const float* pre, float* act, const int32_t* offsets, int64_t num_buckets,
                                  int64_t S, int64_t I, void* stream) {
  MOE_REQUIRE(S >= 0 && S < (1ll << 31) && I > 0 && num_buckets >= 1, MOE_ERR_INVALID, "f32 swiglu: bad sizes");
  if (S == 0) return MOE_OK;
  MOE_REQUIRE(pre && act && offsets, MOE_ERR_INVALID, "f32 swiglu: null pointer");
  hipLaunchKernelGGL(f32_swiglu_fwd_kernel, dim3(rows_grid(S)), dim3(256), 0, as_stream(stream), pre, act,
                     static_cast<int>(S), static_cast<int>(I), offsets + (num_buckets - 1));
  return launch_status("moe_f32_swiglu_fwd");
}

extern "C" int moe_f32_swiglu_bwd(const float* d_act, const float* pre, float* d_pre, const int32_t* offsets,
                                  int64_t num_buckets, int64_t S, int64_t I, void* stream) {
  MOE_REQUIRE(S >= 0 && S < (1ll << 31) && I > 0 && num_buckets >= 1, MOE_ERR_INVALID,
              "f32 swiglu bwd: bad sizes");
  if (S == 0) return MOE_OK;
  MOE_REQUIRE(d_act && pre && d_pre && offsets, MOE_ERR_INVALID, "f32 swiglu bwd: null pointer");
  hipLaunchKernelGGL(f32_swiglu_bwd_kernel, dim3(rows_grid(S)), dim3(256), 0, as_stream(stream), d_act, pre, d_pre,
                     static_cast<int>(S), static_cast<int>(I), offsets + (num_buckets - 1));
  return launch_status("moe_f32_swiglu_bwd");
}

extern "C" int moe_f32_combine_fwd(const float* y, const int32_t* pos_of_slot, const int32_t* offsets,
                                   int64_t num_buckets, const float* scores, int64_t T, int64_t H, int64_t k,
                                   float* out, void* stream) {
  MOE_REQUIRE(T >= 0 && H > 0 && k >= 1 && k <= kMaxSlots && num_buckets >= 1, MOE_ERR_INVALID,
              "f32 combine: bad sizes");
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(y && pos_of_slot && offsets && scores && out, MOE_ERR_INVALID, "f32 combine: null pointer");
  hipLaunchKernelGGL(f32_combine_fwd_kernel, dim3(rows_grid(T)), dim3(256), 0, as_stream(stream), y, pos_of_slot,
                     offsets + (num_buckets - 1), scores, static_cast<int>(T), static_cast<int>(H),
                     static_cast<int>(k), out);
  return launch_status("moe_f32_combine_fwd");
}

extern "C" int moe_f32_combine_bwd(const float* d_out, const float* y, const int32_t* pos_of_slot,
                                   const int32_t* offsets, int64_t num_buckets, const float* scores, int64_t T,
                                   int64_t H, int64_t k, float* d_y, float* d_scores, void* stream) {
  MOE_REQUIRE(T >= 0 && H > 0 && k >= 1 && k <= kMaxSlots && num_buckets >= 1, MOE_ERR_INVALID,
              "f32 combine bwd: bad sizes");
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(d_out && y && pos_of_slot && offsets && scores && d_y && d_scores, MOE_ERR_INVALID,
              "f32 combine bwd: null pointer");
  hipLaunchKernelGGL(f32_combine_bwd_kernel, dim3(rows_grid(T)), dim3(256), 0, as_stream(stream), d_out, y,
                     pos_of_slot, offsets + (num_buckets - 1), scores, static_cast<int>(T), static_cast<int>(H),
                     static_cast<int>(k), d_y, d_scores);
  return launch_status("moe_f32_combine_bwd");
}

extern "C" int moe_f32_permute_bwd(const float* d_xp, const int32_t* pos_of_slot, const int32_t* offsets,
                                   int64_t num_buckets, int64_t T, int64_t H, int64_t k, const float* d_add,
                                   float* d_x, void* stream) {
  MOE_REQUIRE(T >= 0 && H > 0 && k >= 1 && k <= kMaxSlots && num_buckets >= 1, MOE_ERR_INVALID,
              "f32 permute bwd: bad sizes");
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(d_xp && pos_of_slot && offsets && d_x, MOE_ERR_INVALID, "f32 permute bwd: null pointer");
  hipLaunchKernelGGL(f32_permute_bwd_kernel, dim3(rows_grid(T)), dim3(256), 0, as_stream(stream), d_xp, pos_of_slot,
                     offsets + (num_buckets - 1), static_cast<int>(T), static_cast<int>(H), static_cast<int>(k),
                     d_add, d_x);
  return launch_status("moe_f32_permute_bwd");
}
