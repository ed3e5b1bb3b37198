// Router top-k softmax and the Switch load-balancing loss (gfx950).
//
// A token's logits sit in the registers of 16 lanes (up to 256 experts, four
// tokens per wave) or of a whole wave, so softmax statistics and the k-way
// selection are DPP reductions with no LDS.  Selection is on the logits
// (softmax is monotone), largest first, ties to the lower expert index;
// probabilities are exp(l - max) / sum in fp32.
//
// Reference arithmetic: TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267
// (router) and :514-593 (load_balancing_loss_func); the one-rank SP variant is
// parallel/parallel/engine/model_parallel/sequence_parallel.py:239-280.
#include <algorithm>
#include <type_traits>

#include "dma.h"
#include "gemm.h"
#include "router_token.h"

namespace moe {

// k-way selection: sel_idx/sel_logit are the same in all lanes of the token.
template <int LPT, int NPL, int KM>
__device__ __forceinline__ void select_topk(const float (&v)[NPL], int E, int k, int (&sel_idx)[KM],
                                            float (&sel_logit)[KM]) {
  const int sub = Tok<LPT>::sub();
  unsigned taken = 0;  // bit j: item j of this lane already selected
#pragma unroll
  for (int r = 0; r < KM; ++r) {
    if (r < k) {
      float best = -INFINITY;
      int bidx = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int e = sub + j * LPT;
        // Items are visited in increasing e, so ">" keeps the lower index on
        // ties; the first live item is always taken (covers -inf logits).
        // Bitwise operators keep the scan free of branches.
        const bool take = (e < E) & !(taken & (1u << j)) & ((v[j] > best) | (bidx == 0x7fffffff));
        best = take ? v[j] : best;
        bidx = take ? e : bidx;
      }
      tok_argmax<LPT>(best, bidx);
      sel_idx[r] = bidx;
      sel_logit[r] = best;
      if (bidx != 0x7fffffff && (bidx & (LPT - 1)) == sub) taken |= 1u << (bidx / LPT);
    }
  }
}

// Top-k probabilities of the selection, then the scores (renormalised with
// `norm`) and indices: lane r of the token takes selection r (r < k <= LPT),
// and the renormalising total is a sum over the token's lanes.
template <int LPT, int KM>
__device__ __forceinline__ void write_topk(const SoftmaxStats& st, const int (&sel)[KM], const float (&sl)[KM], int k,
                                           int norm, float* __restrict__ scores, int64_t* __restrict__ indices,
                                           int64_t t, bool bf16_scores = false) {
  const int sub = Tok<LPT>::sub();
  int my_idx = 0;
  float my_logit = -INFINITY;
#pragma unroll
  for (int r = 0; r < KM; ++r) {
    if (r < k && sub == r) {
      my_idx = sel[r];
      my_logit = sl[r];
    }
  }
  const bool mine = sub < k;
  const float pv = mine ? expf(my_logit - st.max) / st.sum : 0.0f;
  const float tot = tok_sum<LPT>(pv);
  if (mine) {
    const float sc = norm ? pv / tot : pv;
    scores[t * k + sub] = bf16_scores ? bf16_to_f32(f32_to_bf16(sc)) : sc;
    indices[t * k + sub] = my_idx;
  }
}

template <int LPT, int NPL, int KT>
__global__ __launch_bounds__(kRouterWaves * kWave) void router_topk_fwd_kernel(const float* __restrict__ logits,
                                                                                float* __restrict__ scores,
                                                                                int64_t* __restrict__ indices, int T,
                                                                                int E, int k_rt, int norm) {
  constexpr int KM = KT ? KT : kMaxTopK;
  const int k = KT ? KT : k_rt;
  const int t = blockIdx.x * Tok<LPT>::kPerBlock + Tok<LPT>::slot();
  if (t >= T) return;  // a whole token's lanes leave together
  float v[NPL];
  load_row<LPT>(logits + static_cast<int64_t>(t) * E, E, v);
  const SoftmaxStats st = softmax_stats<LPT>(v);
  int sel[KM];
  float sl[KM];
  select_topk<LPT>(v, E, k, sel, sl);
  write_topk<LPT>(st, sel, sl, k, norm, scores, indices, t);
}

// The block's per-token aux terms (P_e, c_e, W) are summed over its token
// slots in slot order into one partial row (shared by the fused router pass
// and aux_partial_kernel, so that both give the same partials).
template <int LPT, int NPL>
__device__ __forceinline__ void aux_block_partial(float (*part)[2 * LPT * NPL + 1], const float (&P)[NPL],
                                                  const float (&C)[NPL], float W, int E, float* __restrict__ out) {
  const int sub = Tok<LPT>::sub(), slot = Tok<LPT>::slot();
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    if (e < E) {
      part[slot][e] = P[j];
      part[slot][E + e] = C[j];
    }
  }
  if (sub == 0) part[slot][2 * E] = W;
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * E + 1; i += blockDim.x) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < Tok<LPT>::kPerBlock; ++w) s += part[w][i];
    out[i] = s;
  }
}

// One token's routing from its raw logits v (the lane's experts sub + j LPT;
// entries past E are ignored): adds the bias, writes the logits, the top-k
// softmax scores and indices and, with_aux, the token's aux terms (the
// arithmetic of aux_partial_kernel's per-slot sums, which start from zero).
// With logits_b, the logits are those of a bf16 linear (the reference under
// bf16 autocast, parallel/parallel/engine/engine.py:141): rounded to bf16
// (after the bias) before the fp32 softmax and top-k, written to logits_b as
// bf16 and to logits as the same values in fp32; the scores are rounded to
// bf16 as the reference's cast to the logits' dtype (modeling_qwen3_moe.py:266).
template <int LPT, int NPL, int KT>
__device__ __forceinline__ void route_token(float (&v)[NPL], int64_t t, int E, int k, int norm,
                                            const float* __restrict__ bias, float* __restrict__ logits,
                                            bf16_t* __restrict__ logits_b, float* __restrict__ scores,
                                            int64_t* __restrict__ indices, const float* __restrict__ token_weight,
                                            bool with_aux, float (&P)[NPL], float (&C)[NPL], float& W) {
  constexpr int KM = KT ? KT : kMaxTopK;
  const int sub = Tok<LPT>::sub();
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    if (e < E) {
      if (bias) v[j] += bias[e];
      if (logits_b) {
        const bf16_t b = f32_to_bf16(v[j]);
        v[j] = bf16_to_f32(b);
        logits_b[t * E + e] = b;
      }
      logits[t * E + e] = v[j];
    } else {
      v[j] = -INFINITY;
    }
  }
  const SoftmaxStats st = softmax_stats<LPT>(v);
  int sel[KM];
  float sl[KM];
  select_topk<LPT>(v, E, k, sel, sl);
  write_topk<LPT>(st, sel, sl, k, norm, scores, indices, t, logits_b != nullptr);
  if (with_aux) {
    const float w = token_weight ? token_weight[t] : 1.0f;
    W = 0.0f + w;
    const float inv_sum = 1.0f / st.sum;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int e = sub + j * LPT;
      if (e < E) {
        P[j] = 0.0f + w * (expf(v[j] - st.max) * inv_sum);
        float cnt = 0.0f;
#pragma unroll
        for (int r = 0; r < KM; ++r)
          if (r < k && sel[r] == e) cnt += 1.0f;
        C[j] = 0.0f + w * cnt;
      }
    }
  }
}

// logits[t] = sum_s partials[s][t] (+ bias), then the top-k softmax of that row.
// With aux_ws, also the aux-loss partials of the block's tokens from the
// same softmax and selection (the layout and arithmetic of aux_partial_kernel).
template <int LPT, int NPL, int KT>
__global__ __launch_bounds__(kRouterWaves * kWave) void router_reduce_topk_kernel(
    const float* __restrict__ partials, int splits, const float* __restrict__ bias, float* __restrict__ logits,
    bf16_t* __restrict__ logits_b, float* __restrict__ scores, int64_t* __restrict__ indices, int T, int E, int k_rt,
    int norm, const float* __restrict__ token_weight, float* __restrict__ aux_ws) {
  const int k = KT ? KT : k_rt;
  __shared__ float part[Tok<LPT>::kPerBlock][2 * LPT * NPL + 1];  // E <= LPT NPL
  const int sub = Tok<LPT>::sub();
  const int t = blockIdx.x * Tok<LPT>::kPerBlock + Tok<LPT>::slot();
  if (t >= T && !aux_ws) return;
  const int64_t plane = static_cast<int64_t>(T) * E;
  float P[NPL], C[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) P[j] = C[j] = 0.0f;
  float W = 0.0f;
  if (t < T) {
    float v[NPL];
    // All of the lane's split loads are issued before any add; the adds go
    // in split order.
#pragma unroll
    for (int j = 0; j < NPL; ++j) v[j] = 0.0f;
    int sp = 0;
    for (; sp + 8 <= splits; sp += 8) {
      float q[8][NPL];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          const int e = sub + j * LPT;
          q[u][j] = e < E ? partials[(sp + u) * plane + static_cast<int64_t>(t) * E + e] : 0.0f;
        }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int j = 0; j < NPL; ++j) v[j] += q[u][j];
    }
    for (; sp < splits; ++sp) {
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int e = sub + j * LPT;
        v[j] += e < E ? partials[sp * plane + static_cast<int64_t>(t) * E + e] : 0.0f;
      }
    }
    route_token<LPT, NPL, KT>(v, t, E, k, norm, bias, logits, logits_b, scores, indices, token_weight,
                              aux_ws != nullptr, P, C, W);
  }  // t < T
  if (aux_ws) aux_block_partial<LPT>(part, P, C, W, E, aux_ws + static_cast<int64_t>(blockIdx.x) * (2 * E + 1));
}

// The router GEMM, reduction, top-k softmax and aux partials in one pass, for
// E <= 128 experts with E a multiple of 16.  A block takes the 16 tokens of
// the 16-lane token layout (4 waves x 4 tokens).  Their logits
// x[16 tokens, H] . wr[E, H]^T run on v_mfma_f32_16x16x32_bf16 (A: the token
// rows, B: 16 experts; lane l holds row l % 16, k 8 (l / 16) .. + 7 of a
// 32-deep k-step, and D row 4 (l / 16) + i, column l % 16).
//
// wr reaches LDS by DMA in 128-deep k-chunks: the chunk's 16 NPL wr rows
// (256 bytes each; rows past E and k past H read as zeros) fill a ring stage
// with 1 KiB instructions of 4 whole rows each.  Every block reads all of wr
// from L2, so the DMA keeps every cache line it touches whole: loading the
// MFMA operand layout straight from memory (16 rows x 64 bytes per
// instruction) moved wr at a third of the rate.  x, read once from HBM, is
// loaded straight into the A-operand registers, all of a wave's k-steps at
// once (up to kFusedXSteps of them), so its HBM latency is paid once per
// block rather than once per ring turn.  Wave w multiplies the 32-deep
// k-step w of every chunk (k-steps w, w + 4, ...); the four wave partials
// are added in wave order through LDS, and each token then goes through
// route_token as in router_reduce_topk_kernel.  No split-K partials reach
// memory.
//
// LDS layout of a stage: wr row e at e * 256 bytes, its 16-byte chunk c at
// slot c ^ (e % 16), so that the 16 lanes of a ds_read_b128 pass (16 rows,
// one chunk) touch all 64 banks.
constexpr int kFusedTokens = 16;
constexpr int kFusedChunk = 128;   // k per ring stage (one 32-deep k-step per wave)
constexpr int kFusedXSteps = 32;   // x k-steps x row tiles a wave holds in registers at once

template <int NPL>
struct FusedRing {
  static constexpr int kRows = 16 * NPL;  // wr rows of a stage
  static constexpr int kStageBytes = kRows * kFusedChunk * 2;
  static constexpr int kStages = kStageBytes * 4 <= 160 * 1024 ? 4 : 3;  // E <= 128: 4
  static constexpr int kInst = kStageBytes / 1024;  // DMA instructions per stage
  static constexpr int kPerWave = kInst / kRouterWaves;
  static_assert(kInst % kRouterWaves == 0, "a stage's DMA splits evenly over the waves");
};

template <int NPL, int KT, int MT>
__global__ __launch_bounds__(kRouterWaves * kWave) void router_fused_fwd_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ wr, const float* __restrict__ bias,
    float* __restrict__ logits, bf16_t* __restrict__ logits_b, float* __restrict__ scores,
    int64_t* __restrict__ indices, int T, int H, int E, int k_rt, int norm, const float* __restrict__ token_weight,
    float* __restrict__ aux_ws) {
  constexpr int LPT = 16;
  constexpr int NE = NPL;           // 16-expert tiles covered (E <= 16 NPL)
  constexpr int ROW = 16 * NE + 4;  // padded row of the wave partials: the four 4-token row groups hit distinct banks
  using R = FusedRing<NPL>;
  // Four row tiles of 128 experts hold 128 accumulator registers: the x
  // group is halved there, or the compiler parks x registers in AGPRs while
  // their loads are still in flight (tests/test_asm_hazards.py checks every
  // instantiation's assembly for such early uses).
  constexpr int S = R::kStages, PW = R::kPerWave, XS = kFusedXSteps / MT / (MT * NPL >= 32 ? 2 : 1);
  static_assert(Tok<LPT>::kPerBlock == kFusedTokens, "a block's token slots are the MFMA tile's 16 rows");
  static_assert((kRouterWaves * kFusedTokens * ROW + kFusedTokens * (2 * LPT * NPL + 1)) * 4 <= S * R::kStageBytes,
                "the wave partials and the aux rows fit in the ring once it is drained");
  const int k = KT ? KT : k_rt;
  __shared__ __attribute__((aligned(1024))) char ring[S * R::kStageBytes];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int t0 = blockIdx.x * kFusedTokens * MT;  // MT row tiles of 16 tokens
  constexpr uint32_t kOut = 0x80000000u;  // >= both resource sizes (checked on the host)
  const u32x4_t rw = rsrc_words(wr, static_cast<uint32_t>(E) * static_cast<uint32_t>(H) * 2u);
  const u32x4_t rx = rsrc_words(x, static_cast<uint32_t>(T) * static_cast<uint32_t>(H) * 2u);
  // This wave's DMA instructions j < PW fill stage bytes 1024 (wave PW + j)
  // onwards, wr rows 4 (wave PW + j) + lane / 16; per lane the row's byte
  // offset (kOut for a row past E) and the k of its chunk within a k-chunk.
  uint32_t dbase[PW];
  int dk[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int r = 4 * (wave * PW + j) + lane / 16;
    dk[j] = 8 * ((lane & 15) ^ (r & 15));
    dbase[j] = r < E ? static_cast<uint32_t>(r) * static_cast<uint32_t>(H) * 2u : kOut;
  }
  const uint32_t ring_lds = lds_address(ring);
  const int nch = (H + kFusedChunk - 1) / kFusedChunk;
  auto issue = [&](int c, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      // H % 8 == 0: a lane's 8 k are all inside or all outside.  Past the
      // last chunk kk >= H; a row past E stays out of range (kOut plus less
      // than E H 2 bytes).
      const int kk = c * kFusedChunk + dk[j];
      const uint32_t off = kk < H ? dbase[j] + static_cast<uint32_t>(kk) * 2u : kOut;
      dma16(rw, off, __builtin_amdgcn_readfirstlane(ring_lds + st * R::kStageBytes + (wave * PW + j) * 1024));
    }
  };
  // A operand of row tile m: x row t0 + 16 m + l % 16, k 8 (l / 16) .. + 7
  // of k-step 4 c + wave.
  const int r16 = lane & 15;
  auto x_off = [&](int c, int m) __attribute__((always_inline)) {
    const int t = t0 + 16 * m + r16;
    const int kk = (4 * c + wave) * 32 + 8 * (lane >> 4);
    return (t < T && kk < H) ? static_cast<uint32_t>(t) * static_cast<uint32_t>(H) * 2u + static_cast<uint32_t>(kk) * 2u
                             : kOut;
  };
  // B operand (tile n): wr row 16 n + l % 16, chunk 4 wave + l / 16.
  const int frag = r16 * 256 + (((4 * wave + (lane >> 4)) ^ r16) << 4);
  f32x4_t acc[MT][NE];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < NE; ++n) acc[m][n] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // The multiply of k-chunk c reads its wr fragments one iteration ahead:
  // iteration c waits for chunk c + 1 (this wave's DMA, all but the S - 3
  // younger chunks, then every wave's through the barrier), refills the
  // stage of chunk c - 1 (whose fragments were consumed by iteration c - 1's
  // MFMAs, before the barrier) with chunk c + S - 1, reads chunk c + 1's
  // fragments and multiplies chunk c's.
  static_assert(S >= 3, "the fragment prefetch needs a stage between the one read and the one refilled");
  static_assert((XS - 1) * MT >= (S - 3) * PW && XS >= S - 2,
                "at every k-step the wait leaves in flight only loads younger than the step's x registers");
  bf16x8_t bq[NE];
  for (int g0 = 0; g0 < nch; g0 += XS) {
    // The x loads are inline assembly like the DMA, so that the compiler
    // adds no waits of its own (it would count them without the DMA issued
    // after them and drain the ring); each k-step's wait below names the
    // register it makes ready.
    u32x4_t xa[XS][MT];
#pragma unroll
    for (int q = 0; q < XS; ++q)
#pragma unroll
      for (int m = 0; m < MT; ++m)
        asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, 0 offen"
                     : "=v"(xa[q][m])
                     : "v"(g0 + q < nch ? x_off(g0 + q, m) : kOut), "s"(rx)
                     : "memory");
    if (g0 == 0) {
#pragma unroll
      for (int s = 0; s < S - 1; ++s) issue(s, s);
      wait_vmcnt<(S - 2) * PW>();  // chunk 0 (and the x loads before it)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
#pragma unroll
      for (int n = 0; n < NE; ++n) bq[n] = *reinterpret_cast<const bf16x8_t*>(ring + 16 * n * 256 + frag);
    }
#pragma unroll
    for (int q = 0; q < XS; ++q) {
      const int c = g0 + q;
      if (c >= nch) break;
      const int cst = c % S;
      // The x loads of group 0 precede every DMA; a later group's follow the
      // DMA of chunks up to g0 + S - 2, and at k-step q at least
      // (XS - 1 - q) MT x loads and q PW DMA instructions are younger than
      // xa[q][*], never fewer than the S - 3 chunks the wait leaves in
      // flight: xa[q][*] are ready.
      asm volatile("s_waitcnt vmcnt(%1)" : "+v"(xa[q][0]) : "n"((S - 3) * PW) : "memory");
#pragma unroll
      for (int m = 1; m < MT; ++m) asm volatile("" : "+v"(xa[q][m]));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      issue(c + S - 1, cst == 0 ? S - 1 : cst - 1);
      const char* nst = ring + (cst + 1 == S ? 0 : cst + 1) * R::kStageBytes;
      bf16x8_t bn[NE];
#pragma unroll
      for (int n = 0; n < NE; ++n) bn[n] = *reinterpret_cast<const bf16x8_t*>(nst + 16 * n * 256 + frag);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, xa[q][m]);
#pragma unroll
        for (int n = 0; n < NE; ++n)  // (tiles past E multiply the zeros their rows read)
          acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[n], acc[m][n], 0, 0, 0);
      }
#pragma unroll
      for (int n = 0; n < NE; ++n) bq[n] = bn[n];
    }
  }
  wait_vmcnt<0>();  // the trailing DMA (zeros) lands before the ring is reused
  auto wpart = reinterpret_cast<float (*)[kFusedTokens][ROW]>(ring);
  auto part = reinterpret_cast<float (*)[2 * LPT * NPL + 1]>(ring + kRouterWaves * kFusedTokens * ROW * 4);
  const int sub = Tok<LPT>::sub(), slot = Tok<LPT>::slot();
  const int rows = (T + kFusedTokens - 1) / kFusedTokens;  // aux partial rows: one per 16 tokens
  // One row tile at a time through the wave partials: the barrier first
  // retires the ring's last reads (m = 0) or the previous tile's reads of
  // the partials and aux rows.
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NE; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) wpart[wave][4 * (lane >> 4) + i][16 * n + r16] = acc[m][n][i];
    __syncthreads();
    const int t = t0 + 16 * m + slot;
    float P[NPL], C[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) P[j] = C[j] = 0.0f;
    float W = 0.0f;
    if (t < T) {
      float v[NPL];
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int e = sub + j * LPT;
        v[j] = ((wpart[0][slot][e] + wpart[1][slot][e]) + wpart[2][slot][e]) + wpart[3][slot][e];
      }
      route_token<LPT, NPL, KT>(v, t, E, k, norm, bias, logits, logits_b, scores, indices, token_weight,
                                aux_ws != nullptr, P, C, W);
    }
    const int row = blockIdx.x * MT + m;  // block-uniform
    if (aux_ws && row < rows) aux_block_partial<LPT>(part, P, C, W, E, aux_ws + static_cast<int64_t>(row) * (2 * E + 1));
  }
}

// out[i] = bf16(sum_c partials[c][i]) over n elements, fixed order; with
// accumulate, out[i] = bf16(out[i] + bf16(sum)), torch's bf16 add of a fresh
// gradient into an existing one.
__global__ void reduce_partials_bf16_kernel(const float* __restrict__ partials, int chunks, int64_t n,
                                            bf16_t* __restrict__ out, int accumulate) {
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x * 4) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c = 0; c < chunks; ++c) {
      float4 v = *reinterpret_cast<const float4*>(partials + c * n + i);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    if (accumulate) {
      const uint2 old = *reinterpret_cast<const uint2*>(out + i);
      acc.x = bf16_to_f32(f32_to_bf16(acc.x)) + lo_bf16(old.x);
      acc.y = bf16_to_f32(f32_to_bf16(acc.y)) + hi_bf16(old.x);
      acc.z = bf16_to_f32(f32_to_bf16(acc.z)) + lo_bf16(old.y);
      acc.w = bf16_to_f32(f32_to_bf16(acc.w)) + hi_bf16(old.y);
    }
    uint2 o;
    o.x = pack_bf16x2(acc.x, acc.y);
    o.y = pack_bf16x2(acc.z, acc.w);
    *reinterpret_cast<uint2*>(out + i) = o;
  }
}

// d_logits = p * (dp - <dp, p>) (+ d_add), dp scattered from the (renormalised)
// top-k; the f32 result goes to d_logits and its bf16 rounding to
// d_logits_bf16 (either may be null).  d_add may alias d_logits.  With
// aux_stats, the aux loss's logits gradient is added as well, computed as
// aux_bwd_kernel computes it (from the same softmax) and added where d_add
// would be: the result is the bits of aux_bwd_kernel's output passed as
// d_add.
//
// With bf16_terms (the bf16-logit router) the logits are a bf16 tensor in the
// reference (the router linear under bf16 autocast), and autograd sums the
// gradients its consumers return, each already bf16, in bf16: the softmax
// path's gradient and the aux term are rounded to bf16 first and every sum
// is rounded again, as bf16(bf16(softmax path) + bf16(bf16(aux) + d_add)),
// d_add holding a bf16 gradient's values.
template <int LPT, int NPL, int KT>
__global__ __launch_bounds__(kRouterWaves * kWave) void router_topk_bwd_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ indices, const float* __restrict__ d_scores, int T,
    int E, int k_rt, int norm, const float* d_add, float* d_logits, bf16_t* __restrict__ d_logits_bf16,
    const float* __restrict__ token_weight, const float* __restrict__ aux_stats, const float* __restrict__ d_aux,
    int bf16_terms) {
  using Row = TopkBwdRow<LPT, NPL, KT>;
  const int k = KT ? KT : k_rt;
  int t = blockIdx.x * Tok<LPT>::kPerBlock + Tok<LPT>::slot();
  if constexpr (LPT == kWave) t = __builtin_amdgcn_readfirstlane(t);  // one token per wave: scalar route loads
  if (t >= T) return;
  Row row;
  topk_bwd_load(row, logits, indices, d_add, t, E, k, token_weight, aux_stats, d_aux);
  float ds[Row::KM];
#pragma unroll
  for (int q = 0; q < Row::KM; ++q) ds[q] = q < k ? d_scores[static_cast<int64_t>(t) * k + q] : 0.0f;
  topk_bwd_finish(row, ds, logits, t, E, k, norm, d_add != nullptr, aux_stats != nullptr, d_logits, d_logits_bf16,
                  bf16_terms);
}

// ------------------------------------------------------------------ aux loss

constexpr int kAuxGroups = 16;  // row groups of the partial reduction

// Lanes per token for E experts, and tokens per block.
constexpr int lanes_per_token(int64_t E) { return E <= 16 * kMaxPerLane ? 16 : kWave; }
constexpr int tokens_per_block(int64_t E) { return kRouterWaves * (kWave / lanes_per_token(E)); }

// One partial row per block of tokens_per_block(E) tokens, as the router
// kernels write them, so that the standalone loss sums the same rows in the
// same groups and gives their bits at any T.
int aux_blocks(int64_t T, int64_t E) {
  const int64_t tpb = tokens_per_block(E);
  int64_t b = (T + tpb - 1) / tpb;
  if (b < 1) b = 1;
  return static_cast<int>(b);
}

// Per block partials: ws[b] = (P_0..P_{E-1}, c_0..c_{E-1}, W), fixed-order sums.
template <int LPT, int NPL, int KT>
__global__ __launch_bounds__(kRouterWaves * kWave) void aux_partial_kernel(const float* __restrict__ logits,
                                                                            const float* __restrict__ token_weight,
                                                                            int T, int E, int k_rt,
                                                                            float* __restrict__ ws) {
  constexpr int KM = KT ? KT : kMaxTopK;
  const int k = KT ? KT : k_rt;
  __shared__ float part[Tok<LPT>::kPerBlock][2 * LPT * NPL + 1];  // E <= LPT NPL
  const int sub = Tok<LPT>::sub();
  float P[NPL], C[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) P[j] = C[j] = 0.0f;
  float W = 0.0f;
  const int stride = gridDim.x * Tok<LPT>::kPerBlock;
  for (int t = blockIdx.x * Tok<LPT>::kPerBlock + Tok<LPT>::slot(); t < T; t += stride) {
    float v[NPL];
    load_row<LPT>(logits + static_cast<int64_t>(t) * E, E, v);
    const SoftmaxStats st = softmax_stats<LPT>(v);
    int sel[KM];
    float sl[KM];
    select_topk<LPT>(v, E, k, sel, sl);
    const float w = token_weight ? token_weight[t] : 1.0f;
    W += w;
    const float inv_sum = 1.0f / st.sum;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int e = sub + j * LPT;
      if (e < E) {
        P[j] += w * (expf(v[j] - st.max) * inv_sum);
        float cnt = 0.0f;
#pragma unroll
        for (int r = 0; r < KM; ++r)
          if (r < k && sel[r] == e) cnt += 1.0f;
        C[j] += w * cnt;
      }
    }
  }
  aux_block_partial<LPT>(part, P, C, W, E, ws + static_cast<int64_t>(blockIdx.x) * (2 * E + 1));
}

// Column sums of the per-block partials in kAuxGroups row groups, fixed
// order: block (x, g) sums entries 64x .. 64x+63 over the rows of group g
// (wave w adds rows w, w+4, ... of the group; the 4 wave sums are combined in
// wave order) into sums[g][entry].
__global__ __launch_bounds__(256) void aux_reduce_kernel(const float* __restrict__ ws, int nblk, int n,
                                                         float* __restrict__ sums) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int entry = blockIdx.x * 64 + lane;
  const int g = blockIdx.y;
  const int per = (nblk + kAuxGroups - 1) / kAuxGroups;
  const int r0 = g * per, r1 = min(nblk, r0 + per);
  float acc = 0.0f;
  if (entry < n) {
#pragma unroll 8
    for (int b = r0 + wave; b < r1; b += 4) acc += ws[static_cast<int64_t>(b) * n + entry];
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && entry < n)
    sums[static_cast<int64_t>(g) * n + entry] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
}

// sums[g] = (P_0..P_{E-1}, c_0..c_{E-1}, W) per row group, added in group
// order -> stats = (c, W), aux = E * sum_e (c_e/W)(P_e/W).
__global__ __launch_bounds__(1024) void aux_finalize_kernel(const float* __restrict__ sums, int E,
                                                             float* __restrict__ stats, float* __restrict__ aux) {
  __shared__ float terms[1024];
  const int tid = threadIdx.x;
  const int n = 2 * E + 1;
  auto total = [&](int entry) {
    float q[kAuxGroups];
#pragma unroll
    for (int g = 0; g < kAuxGroups; ++g) q[g] = sums[static_cast<int64_t>(g) * n + entry];
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < kAuxGroups; ++g) s += q[g];
    return s;
  };
  const float W = total(2 * E);
  float term = 0.0f;
  if (tid < E) {
    float P = total(tid), C = total(E + tid);
    stats[tid] = C;
    term = (C / W) * (P / W);
  }
  if (tid == 0) stats[E] = W;
  terms[tid] = term;
  __syncthreads();
  for (int s = 512; s >= 1; s >>= 1) {
    if (tid < s) terms[tid] += terms[tid + s];
    __syncthreads();
  }
  if (tid == 0) aux[0] = static_cast<float>(E) * terms[0];
}

namespace {
// The aux loss from per-block partial rows: the row-group sums, then the loss.
int aux_reduce_finalize(float* ws, int nblk, int64_t E, float* stats, float* aux, hipStream_t st, const char* name) {
  const int n = static_cast<int>(2 * E + 1);
  float* sums = ws + static_cast<int64_t>(nblk) * n;
  hipLaunchKernelGGL(aux_reduce_kernel, dim3((n + 63) / 64, kAuxGroups), dim3(256), 0, st, ws, nblk, n, sums);
  int rc = launch_status(name);
  if (rc) return rc;
  hipLaunchKernelGGL(aux_finalize_kernel, dim3(1), dim3(1024), 0, st, sums, static_cast<int>(E), stats, aux);
  return launch_status(name);
}
}  // namespace

template <int LPT, int NPL>
__global__ __launch_bounds__(kRouterWaves * kWave) void aux_bwd_kernel(const float* __restrict__ logits,
                                                                        const float* __restrict__ token_weight,
                                                                        const float* __restrict__ stats,
                                                                        const float* __restrict__ d_aux, int T, int E,
                                                                        float* __restrict__ d_logits, int accumulate) {
  const int sub = Tok<LPT>::sub();
  const int t = blockIdx.x * Tok<LPT>::kPerBlock + Tok<LPT>::slot();
  if (t >= T) return;
  float v[NPL];
  load_row<LPT>(logits + static_cast<int64_t>(t) * E, E, v);
  const SoftmaxStats st = softmax_stats<LPT>(v);
  const float inv_sum = 1.0f / st.sum;
  const float W = stats[E];
  const float w = token_weight ? token_weight[t] : 1.0f;
  const float scale = d_aux[0] * static_cast<float>(E) * w / (W * W);
  float p[NPL], g[NPL];
  float dot = 0.0f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    p[j] = 0.0f;
    g[j] = 0.0f;
    if (e < E) {
      p[j] = expf(v[j] - st.max) * inv_sum;
      g[j] = scale * stats[e];
      dot += p[j] * g[j];
    }
  }
  dot = tok_sum<LPT>(dot);
  float* drow = d_logits + static_cast<int64_t>(t) * E;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int e = sub + j * LPT;
    if (e < E) {
      float d = p[j] * (g[j] - dot);
      drow[e] = accumulate ? drow[e] + d : d;
    }
  }
}

}  // namespace moe

using namespace moe;

namespace {
// Blocks covering T tokens.
int token_blocks(int64_t T, int64_t E, bool wave_token = false) {
  const int64_t tpb = wave_token ? kRouterWaves : tokens_per_block(E);
  return static_cast<int>((T + tpb - 1) / tpb);
}

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
  if (T == 0) return MOE_OK;  // no tokens: empty buffers may be NULL
  MOE_REQUIRE(logits && scores && indices, MOE_ERR_INVALID, "router topk: null pointer");
  int blocks = token_blocks(T, E);
  with_npl_k(E, k, [&](auto L, auto N, auto K) {
    hipLaunchKernelGGL((router_topk_fwd_kernel<decltype(L)::value, decltype(N)::value, decltype(K)::value>),
                       dim3(blocks),
                       dim3(kRouterWaves * kWave), 0, as_stream(stream), logits, scores, indices, static_cast<int>(T),
                       static_cast<int>(E), static_cast<int>(k), norm_topk_prob ? 1 : 0);
  });
  return launch_status("moe_router_topk_fwd");
}

extern "C" int moe_router_topk_bwd(const float* logits, const int64_t* indices, const float* d_scores, int64_t T,
                                   int64_t E, int64_t k, int norm_topk_prob, float* d_logits, int accumulate,
                                   void* d_logits_bf16, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(logits && indices && d_scores && d_logits, MOE_ERR_INVALID, "router topk bwd: null pointer");
  int blocks = token_blocks(T, E, true);
  with_npl_k<true>(E, k, [&](auto L, auto N, auto K) {
    hipLaunchKernelGGL((router_topk_bwd_kernel<decltype(L)::value, decltype(N)::value, decltype(K)::value>),
                       dim3(blocks),
                       dim3(kRouterWaves * kWave), 0, as_stream(stream), logits, indices, d_scores,
                       static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), norm_topk_prob ? 1 : 0,
                       accumulate ? d_logits : nullptr, d_logits, static_cast<bf16_t*>(d_logits_bf16), nullptr,
                       nullptr, nullptr, 0);
  });
  return launch_status("moe_router_topk_bwd");
}

namespace {
int topk_bwd_bf16(const float* logits, const int64_t* indices, const float* d_scores, const float* d_add,
                  const float* token_weight, const float* stats, const float* d_aux, int64_t T, int64_t E, int64_t k,
                  int norm_topk_prob, void* d_logits_bf16, int bf16_terms, void* stream, const char* name) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(logits && indices && d_scores && d_logits_bf16, MOE_ERR_INVALID, "%s: null pointer", name);
  MOE_REQUIRE(!stats == !d_aux, MOE_ERR_INVALID, "%s: stats and d_aux go together", name);
  int blocks = token_blocks(T, E, true);
  with_npl_k<true>(E, k, [&](auto L, auto N, auto K) {
    hipLaunchKernelGGL((router_topk_bwd_kernel<decltype(L)::value, decltype(N)::value, decltype(K)::value>),
                       dim3(blocks),
                       dim3(kRouterWaves * kWave), 0, as_stream(stream), logits, indices, d_scores,
                       static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), norm_topk_prob ? 1 : 0,
                       d_add, nullptr, static_cast<bf16_t*>(d_logits_bf16), token_weight, stats, d_aux, bf16_terms);
  });
  return launch_status(name);
}
}  // namespace

extern "C" int moe_router_topk_bwd_bf16(const float* logits, const int64_t* indices, const float* d_scores,
                                        const float* d_add, int64_t T, int64_t E, int64_t k, int norm_topk_prob,
                                        void* d_logits_bf16, void* stream) {
  return topk_bwd_bf16(logits, indices, d_scores, d_add, nullptr, nullptr, nullptr, T, E, k, norm_topk_prob,
                       d_logits_bf16, 0, stream, "moe_router_topk_bwd_bf16");
}

extern "C" int moe_router_bf16_logits_bwd(const float* logits, const int64_t* indices, const float* d_scores,
                                          const float* d_logits, const float* token_weight, const float* stats,
                                          const float* d_aux, int64_t T, int64_t E, int64_t k, int norm_topk_prob,
                                          void* d_logits_bf16, void* stream) {
  return topk_bwd_bf16(logits, indices, d_scores, d_logits, token_weight, stats, d_aux, T, E, k, norm_topk_prob,
                       d_logits_bf16, 1, stream, "moe_router_bf16_logits_bwd");
}

extern "C" int moe_router_aux_bwd_bf16(const float* logits, const int64_t* indices, const float* d_scores,
                                       const float* d_add, const float* token_weight, const float* stats,
                                       const float* d_aux, int64_t T, int64_t E, int64_t k, int norm_topk_prob,
                                       void* d_logits_bf16, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(logits && indices && d_scores && stats && d_aux && d_logits_bf16, MOE_ERR_INVALID,
              "router aux bwd bf16: null pointer");
  int blocks = token_blocks(T, E, true);
  with_npl_k<true>(E, k, [&](auto L, auto N, auto K) {
    hipLaunchKernelGGL((router_topk_bwd_kernel<decltype(L)::value, decltype(N)::value, decltype(K)::value>),
                       dim3(blocks),
                       dim3(kRouterWaves * kWave), 0, as_stream(stream), logits, indices, d_scores,
                       static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), norm_topk_prob ? 1 : 0,
                       d_add, nullptr, static_cast<bf16_t*>(d_logits_bf16), token_weight, stats, d_aux, 0);
  });
  return launch_status("moe_router_aux_bwd_bf16");
}

extern "C" size_t moe_aux_loss_workspace_bytes(int64_t T, int64_t E) {
  if (T < 0 || E < 1) return 0;
  return static_cast<size_t>(aux_blocks(T, E) + kAuxGroups) * static_cast<size_t>(2 * E + 1) * sizeof(float);
}

extern "C" int moe_aux_loss_fwd(const float* logits, const float* token_weight, int64_t T, int64_t E, int64_t k,
                                float* aux, float* stats, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  MOE_REQUIRE(logits && aux && stats && workspace, MOE_ERR_INVALID, "aux loss: null pointer");
  MOE_REQUIRE(T >= 1, MOE_ERR_INVALID, "aux loss: needs at least one token");
  MOE_REQUIRE(workspace_bytes >= moe_aux_loss_workspace_bytes(T, E), MOE_ERR_WORKSPACE,
              "aux loss: workspace %zu < %zu bytes", workspace_bytes, moe_aux_loss_workspace_bytes(T, E));
  const int nblk = aux_blocks(T, E);
  float* ws = static_cast<float*>(workspace);
  with_npl_k(E, k, [&](auto L, auto N, auto K) {
    hipLaunchKernelGGL((aux_partial_kernel<decltype(L)::value, decltype(N)::value, decltype(K)::value>),
                       dim3(nblk),
                       dim3(kRouterWaves * kWave), 0, as_stream(stream), logits, token_weight, static_cast<int>(T),
                       static_cast<int>(E), static_cast<int>(k), ws);
  });
  rc = launch_status("moe_aux_loss_fwd(partial)");
  if (rc) return rc;
  return aux_reduce_finalize(ws, nblk, E, stats, aux, as_stream(stream), "moe_aux_loss_fwd(reduce)");
}

extern "C" int moe_aux_loss_bwd(const float* logits, const float* token_weight, const float* stats, const float* d_aux,
                                int64_t T, int64_t E, float* d_logits, int accumulate, void* stream) {
  int rc = check_router(T, E, 1);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(logits && stats && d_aux && d_logits, MOE_ERR_INVALID, "aux loss bwd: null pointer");
  int blocks = token_blocks(T, E, true);
  with_npl<true>(E, [&](auto L, auto N) {
    hipLaunchKernelGGL((aux_bwd_kernel<decltype(L)::value, decltype(N)::value>), dim3(blocks),
                       dim3(kRouterWaves * kWave), 0, as_stream(stream), logits, token_weight, stats, d_aux,
                       static_cast<int>(T), static_cast<int>(E), d_logits, accumulate ? 1 : 0);
  });
  return launch_status("moe_aux_loss_bwd");
}

namespace {
// Rows per weight-gradient partial.  At T = 4096, E = 128, H = 2048 chunks
// of 512 rows take the same time as 256 (the GEMM plus the reduce, 41-42 us
// per step) and write and re-read half the f32 partials (8 instead of 16 MB);
// 1024 rows leave too few blocks (52 us).  At T = 16384, 1024-row chunks (16
// partials instead of 32) gave the same total: the GEMM 31 -> 36 us, the
// reduce 11 -> 7 us.
constexpr int kRouterWgradChunk = 512;

void router_split(int64_t T, int64_t H, int64_t E, int& splits, int& k_chunk) {
  // About 256 (M-tile, N-tile, K-split) work items, one per CU.  More splits
  // cover the CUs more evenly but write and re-read more fp32 partials: at
  // T = 4096, E = 128 the GEMM plus the reduction took 34 us with 16 splits,
  // 29 us with 8 and 28 us with 4.
  const int64_t tiles = std::max<int64_t>(1, ((T + 127) / 128) * ((E + 127) / 128));  // T = 0: no tiles
  int64_t want = (256 + tiles - 1) / tiles;
  int64_t max_splits = (H + 63) / 64;
  if (want > max_splits) want = max_splits;
  if (want < 1) want = 1;
  k_chunk = static_cast<int>(((H + want - 1) / want + 63) / 64 * 64);
  splits = static_cast<int>((H + k_chunk - 1) / k_chunk);
}
}  // namespace

namespace {
// The one-pass router kernel covers up to 128 experts in 16-expert MFMA
// tiles (its wr ring holds three or four 128-deep k-chunks of every expert's
// row), with x and wr each under 2 GiB (its buffer resources).
constexpr int kFusedMaxExperts = 128;
bool router_fused(int64_t T, int64_t H, int64_t E) {
  constexpr int64_t kMax = (1ll << 31) - 64;
  return E <= kFusedMaxExperts && E % 16 == 0 && T * H * 2 < kMax && E * H * 2 < kMax;
}

// logits, scores and indices of T >= 1 tokens and, with aux_ws, the aux
// partials of token_blocks(T, E) blocks; `partials` is the split-K workspace
// of the two-pass path (other expert counts).
int route_tokens(const void* x, const void* wr, const float* bias, float* logits, void* logits_bf16, float* scores,
                 int64_t* indices, int64_t T, int64_t H, int64_t E, int64_t k, int norm, const float* token_weight,
                 float* aux_ws, float* partials, hipStream_t st, const char* name) {
  bf16_t* logits_b = static_cast<bf16_t*>(logits_bf16);
  const int blocks = token_blocks(T, E);
  if (router_fused(T, H, E)) {
    // Row tiles of 16 tokens per block: one while the blocks fit the CUs in
    // one round, else two (up to twice the CUs) or four, so that a block's
    // pass over wr (all of it, through L2) serves more tokens rather than
    // the grid taking more rounds.  On 256 CUs, H 2048: 5000-8000 tokens
    // 37 -> 27 us with two tiles, 10000-16000 tokens 53-56 -> 45-46 us with
    // four instead of two.
    const int64_t cus = device_cus(current_device());
    const int mt = blocks > 2 * cus ? 4 : blocks > cus ? 2 : 1;
    const int grid = static_cast<int>((T + kFusedTokens * mt - 1) / (kFusedTokens * mt));
    with_npl_k(E, k, [&](auto, auto N, auto K) {
      if constexpr (16 * decltype(N)::value <= kFusedMaxExperts) {
        auto go = [&](auto M) {
          hipLaunchKernelGGL((router_fused_fwd_kernel<decltype(N)::value, decltype(K)::value, decltype(M)::value>),
                             dim3(grid), dim3(kRouterWaves * kWave), 0, st, static_cast<const bf16_t*>(x),
                             static_cast<const bf16_t*>(wr), bias, logits, logits_b, scores, indices,
                             static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), static_cast<int>(k), norm,
                             token_weight, aux_ws);
        };
        if (mt == 4) go(std::integral_constant<int, 4>{});
        else if (mt == 2) go(std::integral_constant<int, 2>{});
        else go(std::integral_constant<int, 1>{});
      }
    });
    return launch_status(name);
  }
  int splits, k_chunk;
  router_split(T, H, E, splits, k_chunk);
  int rc = router_logits_partials(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), partials,
                                  static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), splits, k_chunk, st);
  if (rc) return rc;
  with_npl_k(E, k, [&](auto L, auto N, auto K) {
    hipLaunchKernelGGL((router_reduce_topk_kernel<decltype(L)::value, decltype(N)::value, decltype(K)::value>),
                       dim3(blocks), dim3(kRouterWaves * kWave), 0, st, partials, splits, bias, logits, logits_b,
                       scores, indices, static_cast<int>(T), static_cast<int>(E), static_cast<int>(k), norm, token_weight,
                       aux_ws);
  });
  return launch_status(name);
}
}  // namespace

extern "C" size_t moe_router_fwd_workspace_bytes(int64_t T, int64_t H, int64_t E) {
  if (T < 0 || H < 1 || E < 1 || router_fused(T, H, E)) return 0;
  int splits, k_chunk;
  router_split(T, H, E, splits, k_chunk);
  return static_cast<size_t>(splits) * static_cast<size_t>(T) * static_cast<size_t>(E) * sizeof(float);
}

extern "C" int moe_router_fwd(const void* x, const void* wr, const float* logit_bias, float* logits,
                              void* logits_bf16, float* scores, int64_t* indices, int64_t T, int64_t H, int64_t E,
                              int64_t k, int norm_topk_prob, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  MOE_REQUIRE(wr && (T == 0 || (x && logits && scores && indices)), MOE_ERR_INVALID, "router fwd: null pointer");
  MOE_REQUIRE(H > 0 && H % 8 == 0 && E % 8 == 0 && aligned16(x) && aligned16(wr), MOE_ERR_UNSUPPORTED,
              "router fwd: H (%lld) and E (%lld) must be multiples of 8 with 16-byte aligned operands",
              (long long)H, (long long)E);
  if (T == 0) return MOE_OK;  // no tokens: empty buffers may be NULL
  const size_t need = moe_router_fwd_workspace_bytes(T, H, E);
  MOE_REQUIRE((workspace || need == 0) && workspace_bytes >= need, MOE_ERR_WORKSPACE,
              "router fwd: workspace %zu < %zu bytes", workspace_bytes, need);
  return route_tokens(x, wr, logit_bias, logits, logits_bf16, scores, indices, T, H, E, k, norm_topk_prob ? 1 : 0,
                      nullptr, nullptr, static_cast<float*>(workspace), as_stream(stream), "moe_router_fwd");
}

extern "C" size_t moe_router_aux_fwd_workspace_bytes(int64_t T, int64_t H, int64_t E) {
  if (T < 0 || H < 1 || E < 1) return 0;
  const int64_t blocks = token_blocks(T, E);
  const size_t aux = static_cast<size_t>(blocks + kAuxGroups) * static_cast<size_t>(2 * E + 1) * sizeof(float);
  return moe_router_fwd_workspace_bytes(T, H, E) + aux;
}

extern "C" int moe_router_aux_fwd(const void* x, const void* wr, const float* logit_bias, const float* token_weight,
                                  float* logits, void* logits_bf16, float* scores, int64_t* indices, int64_t T,
                                  int64_t H, int64_t E, int64_t k, int norm_topk_prob, float* aux, float* stats,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_router(T, E, k);
  if (rc) return rc;
  MOE_REQUIRE(x && wr && logits && scores && indices && aux && stats, MOE_ERR_INVALID,
              "router aux fwd: null pointer");
  MOE_REQUIRE(T >= 1, MOE_ERR_INVALID, "router aux fwd: the aux loss needs at least one token");
  MOE_REQUIRE(H > 0 && H % 8 == 0 && E % 8 == 0 && aligned16(x) && aligned16(wr), MOE_ERR_UNSUPPORTED,
              "router aux fwd: H (%lld) and E (%lld) must be multiples of 8 with 16-byte aligned operands",
              (long long)H, (long long)E);
  const size_t need = moe_router_aux_fwd_workspace_bytes(T, H, E);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE, "router aux fwd: workspace %zu < %zu bytes",
              workspace_bytes, need);
  float* partials = static_cast<float*>(workspace);
  float* aux_ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + moe_router_fwd_workspace_bytes(T, H, E));
  hipStream_t st = as_stream(stream);
  rc = route_tokens(x, wr, logit_bias, logits, logits_bf16, scores, indices, T, H, E, k, norm_topk_prob ? 1 : 0,
                    token_weight, aux_ws, partials, st, "moe_router_aux_fwd(route)");
  if (rc) return rc;
  return aux_reduce_finalize(aux_ws, token_blocks(T, E), E, stats, aux, st, "moe_router_aux_fwd(reduce)");
}

// ---------------------------------------------------------------------------
// The router's backward GEMMs in one pass, for E <= 128 experts (E a multiple
// of 32): dX = dZ . Wr and the split-K partials of dWr = dZ^T . X.
//
// Both products have H as their column dimension and read the same dZ rows.
// A block takes an HN-column slice of H and a chunk of the tokens, and walks
// the chunk 64 tokens at a time: the sub-step's dZ rows (all experts) times
// the block's Wr slice give its dX columns, and dZ^T times the sub-step's X
// slice adds to the block's dWr partial.  dZ is read from L2 once per column
// slice (1 MB at T 4096), X and dX once, the Wr slice once per block.  The
// partials, one fp32 [E, H] plane per token chunk, are added in chunk order by
// reduce_partials_bf16_kernel.
//
// MFMAs are v_mfma_f32_16x16x32_bf16 (A: 16 rows x 32 k, lane l holding row
// l % 16, k 8 (l / 16) .. + 7; B likewise by column; D: lane l holds column
// l % 16, rows 4 (l / 16) .. + 3).  dX is formed transposed, A = the Wr slice
// read as [h][e] and B = the dZ rows, so that each lane's result is 4
// consecutive columns of one token row (8-byte stores).  dWr takes A = dZ^T
// and B = the X slice, both read with ds_read_b64_tr_b16 from their
// token-major tiles: 16 lanes read a 4 (k) x 16 patch, lane i the 4 values of
// row i / 4 at columns 4 (i % 4) .., and each receives the 4 k of column i.
//
// Eight waves in two groups of four (waves w and w + 4 share a SIMD): group g
// takes the sub-steps of parity g, so that one group's MFMAs run while the
// other's LDS reads and DMA are in flight.  Within a group, wave r computes
// dX for tokens 16 r .. + 15 of its sub-step (all HN columns) and the dWr
// rows 32 r .. + 31 (experts) x HN columns.  The groups' dWr sums are added
// through LDS at the end, group 0's first.
//
// LDS: a ring of kRbStages sub-step stages, each a dZ tile [64 tokens][128
// experts] (256-byte rows, 16-byte chunk c of row r at slot c ^ rb_zsw(r)) and
// an X tile [64 tokens][HN] (chunk c of row r at slot c ^ rb_xsw<HN>(r)),
// filled by LDS DMA (1 KiB instructions, lane l -> bytes 16 l ..: each lane
// loads the global chunk that belongs at its slot).  Group g's four waves
// load the sub-steps group g computes.  The Wr slice [128 experts][HN], in the
// X tile's layout, first occupies the two stages the prologue leaves empty and
// is read once into the dX A registers.  With these swizzles the 16 lanes of
// a ds_read_b128 pass and the 32 lanes of a transpose-read pass touch 64
// distinct banks.
namespace moe {

constexpr int kRbTok = 64;            // tokens per sub-step
constexpr int kRbStages = 6;          // ring depth in sub-steps (3 iterations of 2)
constexpr int kRbWaves = 8;
constexpr int kRbE = 128;             // expert rows of the LDS tiles
constexpr int kRbTargetBlocks = 256;  // one block per CU of an MI355X

__device__ __forceinline__ int rb_zsw(int r) {
  r &= 15;
  return ((r & 3) << 2) | (((r >> 3) & 1) << 1) | ((r >> 2) & 1);
}
template <int HN>
__device__ __forceinline__ int rb_xsw(int r) {
  return HN == 32 ? 2 * ((r >> 3) & 1) : 2 * ((r >> 1) & 1) + 4 * ((r >> 3) & 1);
}

template <int HN, int S>
struct RbCfg {
  static_assert(HN == 32 || HN == 64, "column slices of 32 or 64");
  static_assert(S % 2 == 0 && S >= 6, "whole iterations, two of them prefetched");
  static constexpr int kCpr = HN / 8;                // 16-byte chunks per X / Wr row
  static constexpr int kRowsPerInst = 1024 / (HN * 2);
  static constexpr int kZBytes = kRbTok * kRbE * 2;  // 16 KiB
  static constexpr int kXBytes = kRbTok * HN * 2;
  static constexpr int kStage = kZBytes + kXBytes;
  static constexpr int kWBytes = kRbE * HN * 2;
  static constexpr int kZInst = kZBytes / 1024 / 4;  // per wave of the loading group
  static constexpr int kXInst = kXBytes / 1024 / 4;
  static constexpr int kWInst = kWBytes / 1024 / kRbWaves;  // the Wr slice, all eight waves
  static constexpr int kInst = kZInst + kXInst;
  static constexpr int kMT = HN / 16;  // 16-column tiles
  static constexpr int kAhead = S / 2 - 1;  // iterations in flight beyond the current one
  static constexpr int kLds = S * kStage;
  static_assert(kLds <= 160 * 1024, "LDS");
  static_assert(kWBytes <= (S - 2 * kAhead) * kStage, "the Wr slice fits the stages the prologue leaves empty");
  static_assert(4 * (2 * kMT * 4) * 64 * 4 <= kLds, "group 1's dWr sums fit the drained ring");
};

typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

// vmcnt at the end of iteration i: the DMA of the wave's next sub-step (next
// iteration) has landed when at most the younger DMA (A - 1 iterations of NI
// instructions) and the dX stores of the last min(i + 1, A) iterations (MT
// each) are outstanding.
template <int A, int NI, int MT, int C = 1>
__device__ __forceinline__ void rb_wait(int i) {
  static_assert((A - 1) * NI + A * MT < 64, "vmcnt range");
  if constexpr (C == A) {
    wait_vmcnt<(A - 1) * NI + C * MT>();
  } else {
    if (i + 1 == C) wait_vmcnt<(A - 1) * NI + C * MT>();
    else rb_wait<A, NI, MT, C + 1>(i);
  }
}

template <int HN, int S>
__global__ __launch_bounds__(kRbWaves * kWave) void router_bwd_gemm_kernel(
    const bf16_t* __restrict__ dz, const bf16_t* __restrict__ x, const bf16_t* __restrict__ wr,
    bf16_t* __restrict__ dx, float* __restrict__ partials, int T, int H, int E, int tchunk, int nh) {
  using C = RbCfg<HN, S>;
  constexpr int ZI = C::kZInst, XI = C::kXInst, WI = C::kWInst, NI = C::kInst, MT = C::kMT, A = C::kAhead;
  constexpr int RPI = C::kRowsPerInst;
  constexpr uint32_t kOut = 0x80000000u;  // >= every resource size (checked on the host)
  __shared__ __attribute__((aligned(1024))) char lds[C::kLds];
  char* const wtile = lds + 2 * A * C::kStage;  // stages 2 A .. (empty until iteration 0 refills them)
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int grp = wave >> 2, rw = wave & 3;
  const int q = lane >> 4, i16 = lane & 15;
  // Block -> (column slice, token chunk).  Launch indices are dealt to the 8
  // XCDs in turn; each XCD takes a run of consecutive blocks in chunk-major
  // order, so a token chunk's dZ rows are fetched into few L2s (one or two of
  // the eight) and the two blocks reading or writing the halves of a 128-byte
  // X or dX line (HN 32) share an L2.
  const int nb = gridDim.x;
  int b = blockIdx.x;
  if (nb % 8 == 0) b = (b % 8) * (nb / 8) + b / 8;
  const int sp = b / nh, hb = b % nh;
  const int h0 = hb * HN;
  const int tb = sp * tchunk, te = min(T, tb + tchunk);
  const int nit = (te - tb + 2 * kRbTok - 1) / (2 * kRbTok);  // iterations of two sub-steps
  const u32x4_t rz = rsrc_words(dz, static_cast<uint32_t>(T) * static_cast<uint32_t>(E) * 2u);
  const u32x4_t rx = rsrc_words(x, static_cast<uint32_t>(T) * static_cast<uint32_t>(H) * 2u);
  const u32x4_t rwr = rsrc_words(wr, static_cast<uint32_t>(E) * static_cast<uint32_t>(H) * 2u);
  const __amdgpu_buffer_rsrc_t rdx =
      __builtin_amdgcn_make_buffer_rsrc(dx, 0, static_cast<int>(static_cast<uint32_t>(T) * H * 2u), 0x00020000);
  const uint32_t ring = lds_address(lds);
  // This lane's tile row and global column bytes in each of its DMA
  // instructions of a stage (kOut: a chunk past E).
  int zrow[ZI], xrow[XI];
  uint32_t zcol[ZI], xcol[XI];
#pragma unroll
  for (int j = 0; j < ZI; ++j) {
    const int r = 4 * (ZI * rw + j) + q;
    const int c = i16 ^ rb_zsw(r);
    zrow[j] = r;
    zcol[j] = c < E / 8 ? static_cast<uint32_t>(c) * 16u : kOut;
  }
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int r = RPI * (XI * rw + j) + lane / C::kCpr;
    const int c = (lane % C::kCpr) ^ rb_xsw<HN>(r);
    xrow[j] = r;
    xcol[j] = static_cast<uint32_t>(h0 + 8 * c) * 2u;
  }
  // This group's sub-step of iteration it into its stage; past the chunk
  // every lane reads zeros.
  auto issue = [&](int it) __attribute__((always_inline)) {
    const int ss = 2 * it + grp;
    const int t0 = tb + ss * kRbTok;
    const uint32_t base = ring + (ss % S) * C::kStage;
#pragma unroll
    for (int j = 0; j < ZI; ++j) {
      const int t = t0 + zrow[j];
      const uint32_t off = (t < te && zcol[j] != kOut)
                               ? static_cast<uint32_t>(t) * static_cast<uint32_t>(E) * 2u + zcol[j]
                               : kOut;
      dma16(rz, off, __builtin_amdgcn_readfirstlane(base + (ZI * rw + j) * 1024));
    }
#pragma unroll
    for (int j = 0; j < XI; ++j) {
      const int t = t0 + xrow[j];
      const uint32_t off = t < te ? static_cast<uint32_t>(t) * static_cast<uint32_t>(H) * 2u + xcol[j] : kOut;
      dma16(rx, off, __builtin_amdgcn_readfirstlane(base + C::kZBytes + (XI * rw + j) * 1024));
    }
  };
  // The Wr slice (expert rows past E read as zeros), then A iterations.
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int r = RPI * (WI * wave + j) + lane / C::kCpr;
    const int c = (lane % C::kCpr) ^ rb_xsw<HN>(r);
    const uint32_t off = r < E ? static_cast<uint32_t>(r) * static_cast<uint32_t>(H) * 2u +
                                     static_cast<uint32_t>(h0 + 8 * c) * 2u
                               : kOut;
    dma16(rwr, off, __builtin_amdgcn_readfirstlane(lds_address(wtile) + (WI * wave + j) * 1024));
  }
#pragma unroll
  for (int it = 0; it < A; ++it) issue(it);
  wait_vmcnt<(A - 1) * NI>();  // the Wr slice and iteration 0
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // Transpose-read address of (k-row kr, column col) in a [k-rows][cols]
  // tile: the X / Wr layout (HN columns) or the dZ layout (128 columns).
  auto xaddr = [&](int kr, int col) __attribute__((always_inline)) {
    return kr * (HN * 2) + (((col >> 3) ^ rb_xsw<HN>(kr)) << 4) + (col & 7) * 2;
  };
  auto zaddr = [&](int kr, int col) __attribute__((always_inline)) {
    return kr * 256 + (((col >> 3) ^ rb_zsw(kr)) << 4) + (col & 7) * 2;
  };
  auto tr8 = [&](const char* p, int off_lo, int off_hi) __attribute__((always_inline)) {
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + off_lo));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + off_hi));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  // Lane (q, i) of a transpose read takes k-row 8 q + 4 h + i / 4 of its
  // 32-deep k-step and columns 4 (i % 4) .. of its 16-column tile.
  const int tr_kr = 8 * q + (i16 >> 2), tr_col = 4 * (i16 & 3);
  // dX^T A operand: Wr slice column tile m (h0 + 16 m ..), k-step ks (experts 32 ks ..).
  bf16x8_t wa[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      wa[m][ks] = tr8(wtile, xaddr(32 * ks + tr_kr, 16 * m + tr_col), xaddr(32 * ks + tr_kr + 4, 16 * m + tr_col));
  wait_lgkmcnt0();  // every wave's Wr reads are done before iteration 0 refills those stages
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  f32x4_t dw[2][MT];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int n = 0; n < MT; ++n) dw[mi][n] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const bool dw_rows[2] = {32 * rw < E, 32 * rw + 16 < E};  // wave-uniform
  const int zrow_b = 16 * rw + i16;  // this lane's token row of the dX^T B operand
  for (int it = 0; it < nit; ++it) {
    // Refill the stages of iteration it - 1: every wave finished reading them
    // before the barrier that ended iteration it - 1.
    issue(it + A);
    const int ss = 2 * it + grp;
    const char* zt = lds + (ss % S) * C::kStage;
    const char* xt = zt + C::kZBytes;
    // dX^T for the wave's 16 tokens: tile m holds columns h0 + 16 m + 4 q ..
    // + 3 of token zrow_b.
    f32x4_t ax[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) ax[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8_t bz =
          *reinterpret_cast<const bf16x8_t*>(zt + zrow_b * 256 + (((4 * ks + q) ^ rb_zsw(zrow_b)) << 4));
#pragma unroll
      for (int m = 0; m < MT; ++m) ax[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[m][ks], bz, ax[m], 0, 0, 0);
    }
    // dWr rows 32 rw + 16 mi .. (experts) x columns 16 n .. over the 64 tokens.
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8_t za[2], xb[MT];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int col = 32 * rw + 16 * mi + tr_col;
        za[mi] = tr8(zt, zaddr(32 * ks + tr_kr, col), zaddr(32 * ks + tr_kr + 4, col));
      }
#pragma unroll
      for (int n = 0; n < MT; ++n)
        xb[n] = tr8(xt, xaddr(32 * ks + tr_kr, 16 * n + tr_col), xaddr(32 * ks + tr_kr + 4, 16 * n + tr_col));
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        if (dw_rows[mi]) {
#pragma unroll
          for (int n = 0; n < MT; ++n) dw[mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(za[mi], xb[n], dw[mi][n], 0, 0, 0);
        }
    }
    // dX stores, issued by every lane (a token past the chunk stores out of
    // range, which the hardware drops), so each iteration adds MT to vmcnt.
    const int t = tb + ss * kRbTok + zrow_b;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint32_t off = t < te ? (static_cast<uint32_t>(t) * static_cast<uint32_t>(H) +
                                     static_cast<uint32_t>(h0 + 16 * m + 4 * q)) * 2u
                                  : kOut;
      const u32x2_t v = u32x2_t{pack_bf16x2(ax[m][0], ax[m][1]), pack_bf16x2(ax[m][2], ax[m][3])};
      __builtin_amdgcn_raw_buffer_store_b64(v, rdx, off, 0, 0);
    }
    rb_wait<A, NI, MT>(it);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  wait_vmcnt<0>();  // the trailing (zero) DMA has landed: the ring is free
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // Group 1 hands its dWr sums to group 0 through the ring (lane-major, so
  // both sides address the same element), group 0 adds them to its own.
  float* hand = reinterpret_cast<float*>(lds) + rw * (2 * MT * 4 * kWave) + lane;
  if (grp == 1) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int n = 0; n < MT; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) hand[((mi * MT + n) * 4 + i) * kWave] = dw[mi][n][i];
  }
  __syncthreads();
  if (grp == 1) return;
  // dWr partial: lane holds column h0 + 16 n + i16 of expert rows 32 rw + 16 mi + 4 q ..
  float* plane = partials + static_cast<int64_t>(sp) * E * H;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int n = 0; n < MT; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 32 * rw + 16 * mi + 4 * q + i;
        const float v = dw[mi][n][i] + hand[((mi * MT + n) * 4 + i) * kWave];
        if (e < E) plane[static_cast<int64_t>(e) * H + h0 + 16 * n + i16] = v;
      }
}

}  // namespace moe

namespace {
bool router_bwd_fused(int64_t T, int64_t H, int64_t E) {
  constexpr int64_t kMax = (1ll << 31) - 64;
  return E <= kRbE && E % 32 == 0 && H % 32 == 0 && T * H * 2 < kMax && T * E * 2 < kMax && E * H * 2 < kMax;
}
// Column slice, token chunk and chunk count of the one-pass kernel: about
// kRbTargetBlocks blocks.  32-column slices keep the chunks (and the fp32
// partials) fewer; from 8192 tokens 64-column slices halve the passes over dZ
// instead.  Entry point with its reduce, H 2048, E 128: T 4096 17.6 us (32)
// against 20.1 us (64), T 16384 44.0 against 40.9 us, T 8192 / H 4096 43.4
// against 40.3 us.
void router_bwd_plan(int64_t T, int64_t H, int& hn, int& tchunk, int& splits) {
  hn = (H % 64 == 0 && T >= 8192) ? 64 : 32;
  const int64_t nh = H / hn;
  int64_t want = (kRbTargetBlocks + nh / 2) / nh;
  if (want < 1) want = 1;
  int64_t tc = (T + want - 1) / want;
  tc = (tc + kRbTok - 1) / kRbTok * kRbTok;
  if (tc < kRbTok) tc = kRbTok;
  tchunk = static_cast<int>(tc);
  splits = static_cast<int>((T + tc - 1) / tc);
}
}  // namespace

extern "C" size_t moe_router_logits_bwd_workspace_bytes(int64_t T, int64_t H, int64_t E) {
  if (T < 0 || H < 1 || E < 1) return 0;
  int64_t chunks;
  if (router_bwd_fused(T, H, E)) {
    int hn, tchunk, splits;
    router_bwd_plan(T, H, hn, tchunk, splits);
    chunks = splits;
  } else {
    chunks = (T + kRouterWgradChunk - 1) / kRouterWgradChunk;
  }
  if (chunks < 1) chunks = 1;
  return static_cast<size_t>(chunks) * static_cast<size_t>(E) * static_cast<size_t>(H) * sizeof(float);
}

extern "C" int moe_router_logits_bwd(const void* d_logits_bf16, const void* x, const void* wr, void* dx, void* dwr,
                                     int dwr_accumulate, int64_t T, int64_t H, int64_t E, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  // With no tokens only dWr (zeros, or unchanged when accumulating) is
  // written; the empty buffers may be NULL.
  MOE_REQUIRE(wr && dwr && (T == 0 || (d_logits_bf16 && x && dx)), MOE_ERR_INVALID,
              "router logits bwd: null pointer");
  MOE_REQUIRE(T >= 0 && H > 0 && E > 0 && H % 8 == 0 && E % 8 == 0, MOE_ERR_UNSUPPORTED,
              "router logits bwd: H (%lld) and E (%lld) must be multiples of 8", (long long)H, (long long)E);
  MOE_REQUIRE(aligned16(dwr), MOE_ERR_INVALID, "router logits bwd: dwr must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const size_t need = moe_router_logits_bwd_workspace_bytes(T, H, E);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE,
              "router logits bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  float* partials = static_cast<float*>(workspace);
  int chunks;
  if (router_bwd_fused(T, H, E)) {
    int hn, tchunk;
    router_bwd_plan(T, H, hn, tchunk, chunks);
    if (T > 0) {
      const int nh = static_cast<int>(H / hn);
      const dim3 grid(nh * chunks);
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(kRbWaves * kWave), 0, st, static_cast<const bf16_t*>(d_logits_bf16),
                           static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), static_cast<bf16_t*>(dx),
                           partials, static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), tchunk, nh);
      };
      if (hn == 64) go(router_bwd_gemm_kernel<64, kRbStages>);
      else go(router_bwd_gemm_kernel<32, kRbStages>);
      const int rc = launch_status("moe_router_logits_bwd(gemm)");
      if (rc) return rc;
    } else {
      chunks = 0;  // no tokens: the reduction below writes a zero gradient
    }
  } else {
    chunks = static_cast<int>((T + kRouterWgradChunk - 1) / kRouterWgradChunk);
  }
  int rc;
  if (T > 0 && !router_bwd_fused(T, H, E)) {  // with no tokens the reduction below writes a zero gradient
    rc = router_dgrad(static_cast<const bf16_t*>(d_logits_bf16), static_cast<const bf16_t*>(wr),
                      static_cast<bf16_t*>(dx), static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), st);
    if (rc) return rc;
    rc = router_wgrad_partials(static_cast<const bf16_t*>(d_logits_bf16), static_cast<const bf16_t*>(x), partials,
                               static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), chunks,
                               kRouterWgradChunk, st);
    if (rc) return rc;
  }
  const int64_t n = E * H;
  int blocks = static_cast<int>((n / 4 + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(reduce_partials_bf16_kernel, dim3(blocks), dim3(256), 0, st, partials, chunks, n,
                     static_cast<bf16_t*>(dwr), dwr_accumulate ? 1 : 0);
  return launch_status("moe_router_logits_bwd(reduce)");
}
