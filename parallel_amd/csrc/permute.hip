// Token permutation into expert-contiguous (or owner-rank-contiguous) order.
//
// A stable counting sort of the S = T*k routed slots by bucket = id / divisor,
// in two small launches plus one bandwidth-bound row gather:
//   1. count:   each block histograms a CHUNK of slots in LDS (integer
//               atomics, so counts are exact and order-free);
//   2. scatter: each block reads the [blocks x buckets] histogram for its
//               prefix over the blocks before it and the buckets' totals
//               (their scan gives the bucket starts; block 0 writes the
//               per-bucket counts and inclusive offsets), then re-walks its
//               chunk 256 slots at a time: a wave finds equal keys with one
//               ballot per key bit, ranks a slot by the popcount of equal-key
//               lanes below it, and waves are ordered through per-round LDS
//               counters, which keeps the sort stable;
//   3. gather:  one wave per sorted row copies hidden[perm/k] (16-byte lanes).
// Sentinel slots (bucket >= num_buckets) land after every real bucket.
//
// Reference: TF/integrations/moe.py:389-437 (sort/gather/histc/cumsum,
// sentinel handling) and parallel/parallel/engine/model_parallel/
// token_dispatch.py:101-125 (argsort by owner, bincount splits, index_select).
#include "common.h"

namespace moe {

constexpr int kChunk = 512;        // slots per block in count/scatter
constexpr int kPermThreads = 256;  // 4 waves
constexpr int kPerThread = kChunk / kPermThreads;
constexpr int kMaxBuckets = 1024;  // real buckets; +1 for the sentinel bucket

// Bucket = floor(id / divisor) (divisor >= 1), as the reference's owner rule
// (torch.div rounding_mode="floor"); a negative id is below bucket 0 and goes
// to the sentinel bucket with the ids past the last bucket.  (C++ division
// truncates toward zero and would put -1 in bucket 0 for divisor > 1.)
__device__ __forceinline__ int bucket_of(int64_t id, int64_t divisor, int nb) {
  if (id < 0) return nb;
  const int64_t b = id / divisor;
  return b >= nb ? nb : static_cast<int>(b);
}

__global__ __launch_bounds__(kPermThreads) void permute_count_kernel(const int64_t* __restrict__ ids, int S,
                                                                      int64_t divisor, int nb,
                                                                      int32_t* __restrict__ hist) {
  __shared__ int h[kMaxBuckets + 1];
  const int nb1 = nb + 1;
  for (int i = threadIdx.x; i < nb1; i += kPermThreads) h[i] = 0;
  __syncthreads();
  const int begin = blockIdx.x * kChunk;
  const int end = min(begin + kChunk, S);
  // All of the thread's ids in flight at once, then the LDS atomics.
  int64_t id[kPerThread];
#pragma unroll
  for (int r = 0; r < kPerThread; ++r) {
    const int s = begin + r * kPermThreads + threadIdx.x;
    id[r] = s < end ? ids[s] : -1;
  }
#pragma unroll
  for (int r = 0; r < kPerThread; ++r)
    if (begin + r * kPermThreads + static_cast<int>(threadIdx.x) < end) atomicAdd(&h[bucket_of(id[r], divisor, nb)], 1);
  __syncthreads();
  for (int i = threadIdx.x; i < nb1; i += kPermThreads) hist[static_cast<int64_t>(blockIdx.x) * nb1 + i] = h[i];
}

// Each block first places its chunk from the count kernel's histogram
// hist[nblk][nb + 1]: per bucket, the counts of the blocks before it (its
// first position within the bucket) and of all blocks (the bucket's size); an
// exclusive scan of the sizes gives the buckets' starts, the sentinel bucket's
// after every real one.  Block 0 also writes counts[e] and the inclusive
// offsets[e] of the real buckets.  (One launch fewer than a separate scan
// kernel; each block reads the nblk x (nb + 1) histogram from L2.)
__global__ __launch_bounds__(kPermThreads) void permute_scatter_kernel(const int64_t* __restrict__ ids, int S,
                                                                        int64_t divisor, int nb,
                                                                        const int32_t* __restrict__ hist, int nblk,
                                                                        int32_t* __restrict__ counts,
                                                                        int32_t* __restrict__ offsets,
                                                                        int32_t* __restrict__ perm,
                                                                        int32_t* __restrict__ pos_of_slot) {
  __shared__ int running[kMaxBuckets + 1];
  __shared__ int total[kMaxBuckets + 1];
  __shared__ int wave_cnt[kPermThreads / kWave][kMaxBuckets + 1];
  __shared__ int wsum[kPermThreads / kWave];
  const int nb1 = nb + 1;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid >> 6;
  const int begin = blockIdx.x * kChunk;
  const int end = min(begin + kChunk, S);
  // Every round's ids in flight before the first round.
  int64_t id[kPerThread];
#pragma unroll
  for (int r = 0; r < kPerThread; ++r) {
    const int s = begin + r * kPermThreads + tid;
    id[r] = s < end ? ids[s] : -1;
  }
  // Per bucket: the blocks before this one, and all blocks; 32 rows' loads in
  // flight at a time.
  constexpr int kRows = 32;
  const int me = static_cast<int>(blockIdx.x);
  for (int e = tid; e < nb1; e += kPermThreads) {
    int before = 0, all = 0;
    for (int b0 = 0; b0 < nblk; b0 += kRows) {
      int c[kRows];
#pragma unroll
      for (int r = 0; r < kRows; ++r) c[r] = b0 + r < nblk ? hist[static_cast<int64_t>(b0 + r) * nb1 + e] : 0;
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        before += b0 + r < me ? c[r] : 0;
        all += c[r];
      }
    }
    running[e] = before;
    total[e] = all;
#pragma unroll
    for (int w = 0; w < kPermThreads / kWave; ++w) wave_cnt[w][e] = 0;
  }
  __syncthreads();
  // Buckets' starts: thread t scans the real buckets t G .. t G + G - 1
  // (G = ceil(nb / kPermThreads) <= 4) in order, the threads in turn.
  constexpr int kG = (kMaxBuckets + kPermThreads - 1) / kPermThreads;
  const int G = (nb + kPermThreads - 1) / kPermThreads;
  int size[kG];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const int e = tid * G + j;
    size[j] = (j < G && e < nb) ? total[e] : 0;
    sum += size[j];
  }
  const int incl = wave_inclusive_scan(sum);
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  int run = incl - sum, n_valid = 0;
#pragma unroll
  for (int w = 0; w < kPermThreads / kWave; ++w) {
    run += w < wave ? wsum[w] : 0;
    n_valid += wsum[w];
  }
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const int e = tid * G + j;
    if (j < G && e < nb) {
      if (me == 0) {
        counts[e] = size[j];
        offsets[e] = run + size[j];
      }
      running[e] += run;
      run += size[j];
    }
  }
  if (tid == 0) running[nb] += n_valid;
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) < nb1) ++nbits;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int r = 0; r < kPerThread; ++r) {
    const int r0 = begin + r * kPermThreads;
    if (r0 >= end) break;
    const int s = r0 + threadIdx.x;
    const bool live = s < end;
    const int key = live ? bucket_of(id[r], divisor, nb) : 0;
    // Lanes holding the same key: intersect one ballot per key bit.
    unsigned long long match = __ballot(live);
#pragma unroll 1
    for (int b = 0; b < nbits; ++b) {
      unsigned long long set = __ballot(live && ((key >> b) & 1));
      match &= ((key >> b) & 1) ? set : ~set;
    }
    const int rank = __popcll(match & lt_mask);
    const bool leader = live && rank == 0;
    if (leader) wave_cnt[wave][key] = __popcll(match);
    __syncthreads();
    if (live) {
      int pos = running[key] + rank;
      for (int w = 0; w < wave; ++w) pos += wave_cnt[w][key];
      if (pos >= 0 && pos < S) {  // always true for a consistent histogram; never write outside
        perm[pos] = s;
        pos_of_slot[s] = pos;
      }
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&running[key], wave_cnt[wave][key]);
      wave_cnt[wave][key] = 0;
    }
    __syncthreads();
  }
}

// permuted[pos_of_slot[t k + j]] = hidden[t] for the token's slots that sort
// below n_valid, and zeros for its sentinel slots.  pos_of_slot is a
// permutation of [0, S), so every row of permuted is written (rows from
// n_valid on are the sentinels' zeros).  One wave per token reads its row
// once and writes it k times; a gather over perm would read it once per route.
template <int KT>
__global__ __launch_bounds__(kPermThreads) void scatter_rows_kernel(const bf16_t* __restrict__ hidden, int H,
                                                                     const int32_t* __restrict__ pos_of_slot, int T,
                                                                     int S, int k,
                                                                     const int32_t* __restrict__ n_valid_ptr,
                                                                     bf16_t* __restrict__ out) {
  constexpr int KM = KT ? KT : kMaxSlots;
  const int lane = threadIdx.x & (kWave - 1);
  const int n_valid = *n_valid_ptr;
  const int nchunk = H / 8;
  for (int t = blockIdx.x * (kPermThreads / kWave) + (threadIdx.x >> 6); t < T;
       t += gridDim.x * (kPermThreads / kWave)) {
    int pos[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      const bool live = KT ? true : j < k;
      pos[j] = __builtin_amdgcn_readfirstlane(live ? pos_of_slot[static_cast<int64_t>(t) * k + j] : -1);
    }
    const uint4* src = reinterpret_cast<const uint4*>(hidden + static_cast<int64_t>(t) * H);
    // Up to four 16-byte chunks per lane in flight before their stores.
    for (int c0 = lane; c0 < nchunk; c0 += 4 * kWave) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = c0 + u * kWave < nchunk ? src[c0 + u * kWave] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        const int p = pos[j];
        if (p >= 0 && p < S) {  // (always, for a permutation; a wave-uniform guard)
          uint4* dst = reinterpret_cast<uint4*>(out + static_cast<int64_t>(p) * H);
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (c0 + u * kWave < nchunk) dst[c0 + u * kWave] = p < n_valid ? v[u] : make_uint4(0, 0, 0, 0);
        }
      }
    }
  }
}

__global__ void dispatch_meta_kernel(const int64_t* __restrict__ ids, const float* __restrict__ scores,
                                     const int32_t* __restrict__ perm, int S, int64_t divisor, int k,
                                     int64_t* __restrict__ local_ids, float* __restrict__ routed_scores,
                                     int64_t* __restrict__ source_tokens) {
  for (int pos = blockIdx.x * blockDim.x + threadIdx.x; pos < S; pos += gridDim.x * blockDim.x) {
    int s = perm[pos];
    if (source_tokens) source_tokens[pos] = s / k;  // slot s = t k + j of token t (s >= 0)
    if (local_ids) {
      // id - floor(id / divisor) * divisor (the reference's send_experts), in [0, divisor)
      const int64_t id = ids[s];
      const int64_t r = id % divisor;
      local_ids[pos] = r < 0 ? r + divisor : r;
    }
    if (routed_scores) routed_scores[pos] = scores[s];
  }
}

// d_hidden[t] = sum_j d_permuted[pos_of_slot[t*k+j]] (+ d_add[t]); one wave
// per token.  Every live slot's row load is issued before any is added
// (slot order, then d_add); KT as in Slots.
template <int KT>
__global__ __launch_bounds__(kPermThreads) void permute_bwd_kernel(const bf16_t* __restrict__ dperm,
                                                                    const int32_t* __restrict__ pos_of_slot,
                                                                    const int32_t* __restrict__ n_valid_ptr, int T,
                                                                    int H, int k, const bf16_t* __restrict__ d_add,
                                                                    bf16_t* __restrict__ dh) {
  constexpr int KM = Slots<KT>::KM;
  const int lane = threadIdx.x & (kWave - 1);
  const int n_valid = *n_valid_ptr;
  const int nchunk = H / 8;
  for (int t = blockIdx.x * (kPermThreads / kWave) + (threadIdx.x >> 6); t < T;
       t += gridDim.x * (kPermThreads / kWave)) {
    Slots<KT> sl;
    sl.load(pos_of_slot, nullptr, t, k, n_valid);
    for (int c = lane; c < nchunk; c += kWave) {
      uint4 v[KM];
#pragma unroll
      for (int j = 0; j < KM; ++j)
        if (KT || j < k)  // the last read of the permuted rows' gradient
          v[j] = ntload16(reinterpret_cast<const uint4*>(dperm + static_cast<int64_t>(sl.pos[j]) * H) + c);
      uint4 va = make_uint4(0, 0, 0, 0);
      if (d_add) va = reinterpret_cast<const uint4*>(d_add + static_cast<int64_t>(t) * H)[c];
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        if (sl.ok[j]) {
          acc[0] += lo_bf16(v[j].x); acc[1] += hi_bf16(v[j].x);
          acc[2] += lo_bf16(v[j].y); acc[3] += hi_bf16(v[j].y);
          acc[4] += lo_bf16(v[j].z); acc[5] += hi_bf16(v[j].z);
          acc[6] += lo_bf16(v[j].w); acc[7] += hi_bf16(v[j].w);
        }
      }
      if (d_add) {
        acc[0] += lo_bf16(va.x); acc[1] += hi_bf16(va.x);
        acc[2] += lo_bf16(va.y); acc[3] += hi_bf16(va.y);
        acc[4] += lo_bf16(va.z); acc[5] += hi_bf16(va.z);
        acc[6] += lo_bf16(va.w); acc[7] += hi_bf16(va.w);
      }
      uint4 o;
      o.x = pack_bf16x2(acc[0], acc[1]);
      o.y = pack_bf16x2(acc[2], acc[3]);
      o.z = pack_bf16x2(acc[4], acc[5]);
      o.w = pack_bf16x2(acc[6], acc[7]);
      reinterpret_cast<uint4*>(dh + static_cast<int64_t>(t) * H)[c] = o;
    }
  }
}

int row_grid(int64_t rows) {
  int64_t b = (rows + (kPermThreads / kWave) - 1) / (kPermThreads / kWave);
  if (b > 8192) b = 8192;
  return static_cast<int>(b < 1 ? 1 : b);
}

}  // namespace moe

using namespace moe;

extern "C" size_t moe_permute_workspace_bytes(int64_t S, int64_t num_buckets) {
  if (S < 0 || num_buckets < 1) return 0;
  int64_t nblk = (S + kChunk - 1) / kChunk;
  if (nblk < 1) nblk = 1;
  return static_cast<size_t>(nblk) * static_cast<size_t>(num_buckets + 1) * sizeof(int32_t);
}

extern "C" int moe_permute_fwd(const void* hidden, int64_t T, int64_t H, const int64_t* ids, int64_t k,
                               int64_t divisor, int64_t num_buckets, void* permuted, int32_t* perm,
                               int32_t* pos_of_slot, int32_t* counts, int32_t* offsets, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return moe::permute_fwd_run(hidden, T, H, ids, k, divisor, num_buckets, permuted, perm, pos_of_slot, counts,
                              offsets, workspace, workspace_bytes, stream);
}

namespace moe {
// Validates and launches moe_permute_fwd's kernels with the given histogram
// workspace (moe_permute_workspace_bytes(T * k, num_buckets) bytes at least).
int permute_fwd_run(const void* hidden, int64_t T, int64_t H, const int64_t* ids, int64_t k, int64_t divisor,
                    int64_t num_buckets, void* permuted, int32_t* perm, int32_t* pos_of_slot, int32_t* counts,
                    int32_t* offsets, void* workspace, size_t workspace_bytes, void* stream) {
  MOE_REQUIRE(T >= 0 && k >= 1 && k <= 16 && T * k < (1ll << 31), MOE_ERR_INVALID,
              "permute: bad T=%lld k=%lld", (long long)T, (long long)k);
  MOE_REQUIRE(divisor >= 1, MOE_ERR_INVALID, "permute: divisor must be >= 1");
  MOE_REQUIRE(num_buckets >= 1 && num_buckets <= kMaxBuckets, MOE_ERR_UNSUPPORTED,
              "permute: num_buckets=%lld outside [1,%d]", (long long)num_buckets, kMaxBuckets);
  MOE_REQUIRE(counts && offsets && (T == 0 || (ids && perm && pos_of_slot)), MOE_ERR_INVALID, "permute: null pointer");
  MOE_REQUIRE(!permuted || (hidden && H > 0 && H % 8 == 0 && aligned16(hidden) && aligned16(permuted)),
              MOE_ERR_INVALID, "permute: rows need H %% 8 == 0 and 16-byte aligned buffers");
  const int S = static_cast<int>(T * k);
  const int nb = static_cast<int>(num_buckets);
  const size_t need = moe_permute_workspace_bytes(S, num_buckets);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE, "permute: workspace %zu < %zu bytes",
              workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  int32_t* hist = static_cast<int32_t*>(workspace);
  const int nblk = (S + kChunk - 1) / kChunk;
  if (nblk > 0) {
    hipLaunchKernelGGL(permute_count_kernel, dim3(nblk), dim3(kPermThreads), 0, st, ids, S, divisor, nb, hist);
    int rc = launch_status("moe_permute_fwd(count)");
    if (rc) return rc;
  }
  // With no slots one block still writes the zero counts and offsets.
  hipLaunchKernelGGL(permute_scatter_kernel, dim3(nblk > 0 ? nblk : 1), dim3(kPermThreads), 0, st, ids, S, divisor, nb,
                     hist, nblk, counts, offsets, perm, pos_of_slot);
  int rc = launch_status("moe_permute_fwd(scatter)");
  if (rc || nblk == 0) return rc;
  if (permuted) {
    MOE_DISPATCH_K(k, scatter_rows_kernel, dim3(row_grid(T)), dim3(kPermThreads), 0, st,
                   static_cast<const bf16_t*>(hidden), static_cast<int>(H), pos_of_slot, static_cast<int>(T),
                   static_cast<int>(S), static_cast<int>(k), offsets + (nb - 1), static_cast<bf16_t*>(permuted));
    rc = launch_status("moe_permute_fwd(rows)");
  }
  return rc;
}
}  // namespace moe

extern "C" int moe_dispatch_meta(const int64_t* ids, const float* scores, const int32_t* perm, int64_t S,
                                 int64_t divisor, int64_t k, int64_t* local_ids, float* routed_scores,
                                 int64_t* source_tokens, void* stream) {
  MOE_REQUIRE(S >= 0 && S < (1ll << 31) && divisor >= 1 && k >= 1 && k < (1ll << 31), MOE_ERR_INVALID,
              "dispatch meta: bad sizes");
  if (S == 0) return MOE_OK;
  MOE_REQUIRE(ids && perm && (!routed_scores || scores), MOE_ERR_INVALID, "dispatch meta: null pointer");
  int blocks = static_cast<int>((S + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(dispatch_meta_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), ids, scores, perm,
                     static_cast<int>(S), divisor, static_cast<int>(k), local_ids, routed_scores, source_tokens);
  return launch_status("moe_dispatch_meta");
}

extern "C" int moe_permute_bwd(const void* d_permuted, const int32_t* pos_of_slot, const int32_t* offsets,
                               int64_t num_buckets, int64_t T, int64_t H, int64_t k, const void* d_add,
                               void* d_hidden, void* stream) {
  MOE_REQUIRE(T >= 0 && k >= 1 && k <= 16 && H > 0 && H % 8 == 0, MOE_ERR_INVALID,
              "permute bwd: bad sizes T=%lld H=%lld k=%lld", (long long)T, (long long)H, (long long)k);
  MOE_REQUIRE(num_buckets >= 1, MOE_ERR_INVALID, "permute bwd: num_buckets must be >= 1");
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(d_permuted && pos_of_slot && offsets && d_hidden, MOE_ERR_INVALID, "permute bwd: null pointer");
  MOE_REQUIRE(aligned16(d_permuted) && aligned16(d_hidden) && (!d_add || aligned16(d_add)), MOE_ERR_INVALID,
              "permute bwd: buffers must be 16-byte aligned");
  MOE_DISPATCH_K(k, permute_bwd_kernel, dim3(row_grid(T)), dim3(kPermThreads), 0, as_stream(stream),
                     static_cast<const bf16_t*>(d_permuted), pos_of_slot, offsets + (num_buckets - 1),
                     static_cast<int>(T), static_cast<int>(H), static_cast<int>(k),
                     static_cast<const bf16_t*>(d_add), static_cast<bf16_t*>(d_hidden));
  return launch_status("moe_permute_bwd");
}
