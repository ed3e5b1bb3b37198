// Grouped bf16 GEMMs for the MoE expert path on gfx950 (MI355X).
//
// One kernel template covers the three contraction shapes of an expert layer:
//   MG / B K-contiguous   forward      c[r,n]   = sum_k a[r,k] w[g][n,k]
//   MG / B N-contiguous   input grad   da[r,n]  = sum_k dc[r,k] w[g][k,n]
//   KG                    weight grad  dw[g][m,n] = sum_{r in g} dc[r,m] a[r,n]
// MG = groups partition the rows of the activation operand (variable M per
// expert), KG = groups partition the reduction (variable K per expert).
//
// Tiling: WM x WN waves; each wave owns (BM/WM) x (BN/WN) of 32x32 MFMA
// sub-tiles (v_mfma_f32_32x32x16_bf16, fp32 accumulators), its row sub-tiles
// interleaved with the other wave rows'.  The expert GEMMs use 256x256 tiles
// (384x128 when the output is at most 1024 columns wide) on 8 waves (two waves
// per SIMD, one workgroup per CU); the small router GEMMs use 128x128 on 4
// waves.  Operands move from HBM to LDS by DMA (buffer_load_dwordx4 ... lds,
// no register staging) into a 5-deep ring of 32-deep k-tiles that fills
// the 160 KiB of LDS, so three or four k-tiles of loads are in flight while
// one is multiplied; each wave fires its share of a k-tile's DMA between its
// MFMA groups.  At the roughly 256 rows per expert of a training step the
// expert GEMMs sit near the ridge of the roofline (about 256 flop per weight
// byte), and the weights stream from HBM only as fast as the bytes in flight
// per CU allow, so the ring takes all of the LDS: the epilogue stages its
// output through the ring stage it has just multiplied.  Each operand
// keeps its HBM layout in LDS (XOR swizzled): K-contiguous fragments are
// ds_read_b128, M/N-contiguous ones (weights in the input gradient, both
// operands of the weight gradient) are ds_read_b64_tr_b16 transpose reads.
// Buffer loads read zero past the resource size, so ragged rows and the K
// tail need no branches.  Row sub-tiles that lie wholly outside the valid
// rows skip their MFMAs (an expert's rows are split evenly over its m-tiles,
// so most m-tiles are partly filled).
//
// Tiles are mapped to groups on the device from the `offs` cumsum (no host
// sync).  The logical tile order is group-major, then n-tile, then m-tile, so
// consecutive tiles share an expert's weight tile and its activation rows;
// the launch index is remapped so that each XCD (blocks are dealt round-robin
// over the 8 XCDs) gets a contiguous run of logical tiles and the sharing
// happens in that XCD's L2.
#include <algorithm>
#include <type_traits>

#include "dma.h"
#include "gemm.h"

namespace moe {

enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_SWIGLU_FWD = 2, EPI_WGRAD = 4 };
enum { MODE_MG = 0, MODE_KG = 1 };

constexpr int kNumXcd = 8;

struct GemmParams {
  const bf16_t* A;  // MG: [rows, K] (lda);  KG: [rows, M] (lda)
  const bf16_t* B;  // MG: per group (stride_bg) [N, K] or [K, N] (ldb);  KG: [rows, N] (ldb)
  void* C;          // MG: [rows, ldc];  KG: per group (stride_cg) [M, N] (ldc)
  void* C2;         // SWIGLU_FWD: pre-activation [rows, 2N] (may be null)
  const int32_t* offs;
  int G;
  int rows;     // total activation rows (M for MG; sum of K for KG)
  int M, N, K;  // GEMM-internal sizes: MG: M = rows, N out cols, K reduction; KG: M x N output per group
  int64_t lda, ldb, ldc, ldp;
  int64_t stride_bg, stride_cg;
  uint32_t a_bytes;  // bytes addressable through the A buffer resource
  uint32_t b_bytes;  // bytes of one group's B (MG) or of all of B (KG)
  uint32_t c_bytes;  // bytes of the output: all of C (MG), one group's (KG) or one split's (split-K)
  uint32_t c2_bytes;  // SWIGLU_FWD: bytes of the pre-activation output (0 if none)
  int swiglu_I;      // SWIGLU_FWD: intermediate size I (weight rows gate: [0,I), up: [I,2I))
  int accumulate;
  int n_tiles, m_tiles_max;
  int total_tiles;     // exact tile count (grouped MG: worst case; the kernel counts the real ones)
  int k_splits, k_chunk;  // MG without groups: split the reduction, partial outputs stacked
  int64_t split_stride;   // elements between split partials of C
  int chunk_rows;         // KG without offs and G > 1: group g = rows [g*chunk_rows, ...)
  // KG into a rank-major bucket (0 = plain): group g's output starts
  // (g / bucket_rows) * bucket_stride + (g % bucket_rows) * stride_cg
  // elements into C instead of g * stride_cg.
  int bucket_rows;
  int64_t bucket_stride;
  // KG with groups: split the tiles over the XCDs by cost (k-steps plus an
  // epilogue allowance per tile) instead of by count (set by the host when
  // the costs fit in 30 bits).
  int cost_split;
};

// ---------------------------------------------------------------- helpers

// Raw buffer loads: offsets at or past the resource's byte size read as zero
// in hardware, so out-of-range rows and the K tail need no branches.
constexpr uint32_t kOOB = 0x80000000u;  // >= every resource size (host checks < 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// silu(g) = g * sigmoid(g), with the hardware exp and reciprocal (1 ulp).
__device__ __forceinline__ float sigmoid_f(float g) { return __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

// Total tiles over all groups, sum_g n_mult * ceil(cnt_g / BM) (wave-uniform).
template <int BM>
__device__ __forceinline__ int count_tiles(const int32_t* offs, int G, int rows, int n_mult) {
  const int lane = threadIdx.x & (kWave - 1);
  int total = 0;
  for (int c0 = 0; c0 < G; c0 += kWave) {
    int g = c0 + lane;
    int nt = 0;
    if (g < G) {
      int hi = min(max(offs[g], 0), rows);
      int lo = g ? min(max(offs[g - 1], 0), hi) : 0;
      nt = n_mult * ((hi - lo + BM - 1) / BM);
    }
    total += __builtin_amdgcn_readlane(wave_inclusive_scan(nt), kWave - 1);
  }
  return __builtin_amdgcn_readfirstlane(total);
}

// Weight gradients (KG): a tile of group g costs its k-steps, ceil(rows_g /
// BK), plus kEpiSteps for its epilogue.  Returns (split(part),
// split(part + 1)), split(x) being the first tile, in group-major order, whose
// cost start is at least x / kNumXcd of the total (wave-uniform): XCD x takes
// tiles [split(x), split(x + 1)).  Under skewed routing the tiles of the
// heavy experts are many times longer than the rest, and a split by count
// leaves some XCDs long tails.  Returns (-1, -1) when the costs are near
// uniform: the split by count is then as balanced and keeps whole rounds of
// tiles per block.
constexpr int kEpiSteps = 2;
template <int BK>
__device__ int2 kg_cost_split(const int32_t* offs, int G, int rows, int per_group, int part) {
  const int lane = threadIdx.x & (kWave - 1);
  auto tile_cost = [&](int g) {
    if (g >= G) return 0;
    const int hi = min(max(offs[g], 0), rows);
    const int lo = g ? min(max(offs[g - 1], 0), hi) : 0;
    return (hi - lo + BK - 1) / BK + kEpiSteps;
  };
  // Up to kCostChunks x 64 groups, every chunk's offsets are loaded at once
  // (one memory round trip at kernel start instead of one per chunk).
  constexpr int kCostChunks = 4;
  const bool cached = G <= kCostChunks * kWave;
  int tcr[kCostChunks];
#pragma unroll
  for (int c = 0; c < kCostChunks; ++c) tcr[c] = cached ? tile_cost(c * kWave + lane) : 0;
  auto chunk_cost = [&](int c0) {
    int v = 0;
#pragma unroll
    for (int c = 0; c < kCostChunks; ++c)
      if (cached && c0 == c * kWave) v = tcr[c];
    return cached ? v : tile_cost(c0 + lane);
  };
  int total = 0;
  float mx = 0.0f;  // largest tile cost
  for (int c0 = 0; c0 < G; c0 += kWave) {
    const int tc = chunk_cost(c0);
    total += __builtin_amdgcn_readlane(wave_inclusive_scan(per_group * tc), kWave - 1);
    mx = fmaxf(mx, wave_max(static_cast<float>(tc)));
  }
  // Near-uniform costs (the largest within a quarter of the mean): the split
  // by count is as balanced and keeps whole rounds of tiles per block.
  if (4.0f * mx * static_cast<float>(G) * per_group <= 5.0f * static_cast<float>(total)) return make_int2(-1, -1);
  // Both boundaries in one more pass (its loads hit the cache the first filled).
  int t_lo = static_cast<int>(static_cast<int64_t>(total) * part / kNumXcd);
  int t_hi = static_cast<int>(static_cast<int64_t>(total) * (part + 1) / kNumXcd);
  int b_lo = part <= 0 ? 0 : -1, b_hi = part + 1 >= kNumXcd ? G * per_group : -1;
  int base = 0;  // cost of the groups before this chunk
  for (int c0 = 0; c0 < G && (b_lo < 0 || b_hi < 0); c0 += kWave) {
    const int tc = chunk_cost(c0);
    const int incl = wave_inclusive_scan(per_group * tc);
    const int tot = __builtin_amdgcn_readlane(incl, kWave - 1);
    auto locate = [&](int target) {
      const int t = target - base;  // wave-uniform, and t < tot = incl[63]
      const int q = __builtin_amdgcn_readfirstlane(__builtin_ctzll(__ballot(incl > t)));  // first lane past t
      const int before = __builtin_amdgcn_readlane(incl - per_group * tc, q);
      const int cq = __builtin_amdgcn_readlane(tc, q);
      return (c0 + q) * per_group + min((t - before + cq - 1) / cq, per_group);
    };
    if (b_lo < 0 && t_lo - base < tot) b_lo = locate(t_lo);
    if (b_hi < 0 && t_hi - base < tot) b_hi = locate(t_hi);
    base += tot;
  }
  if (b_lo < 0) b_lo = G * per_group;
  if (b_hi < 0) b_hi = G * per_group;
  return make_int2(__builtin_amdgcn_readfirstlane(b_lo), __builtin_amdgcn_readfirstlane(b_hi));
}

// Tile configurations: BK-deep k-tiles staged through a STAGES-deep LDS ring.
// PIPE selects the k-loop:
//   0  every wave reads its fragments, multiplies and fires its share of the
//      DMA in each k-step (block barrier every second k-step);
//   1  the same with the next 16-deep half step's fragments read while the
//      current half step's MFMAs run (one barrier per k-step);
//   2  ping-pong: the two waves of a SIMD take turns, one multiplying a k-step
//      from registers while the other reads the next k-step's fragments and
//      fires DMA (two barriers per k-step).
template <int BM_, int BN_, int BK_, int WM_, int WN_, int STAGES_, int PIPE_ = 0>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, STAGES = STAGES_, PIPE = PIPE_;
  static constexpr int kThreads = 64 * WM * WN;
};
// Expert GEMMs and weight gradients: 160 KiB ring, 8 waves.
using BigTile = TileCfg<256, 256, 32, 2, 4, 5>;
// Expert GEMMs with narrow outputs: 384-row tiles, so that an expert of up to
// 384 rows is one m-tile and its weights stream through LDS once per n-tile;
// 160 KiB ring (5 x 32 KiB, so the block barrier pairs k-steps), 8 waves.
using TallTile = TileCfg<384, 128, 32, 4, 2, 5>;
// Router GEMMs (N = E = 128): 80 KiB ring, 4 waves (two workgroups per CU).
using SmallTile = TileCfg<128, 128, 32, 2, 2, 5>;
// The 256x256 loop with the fragment reads of each 16-deep half step
// overlapping the previous half step's MFMAs.
using BigTileP = TileCfg<256, 256, 32, 2, 4, 5, 1>;
// Experts of up to 320 rows in one m-tile: 320x256 tiles (five 32-row
// sub-tiles per wave, 160 accumulator registers per lane), A staged as 384
// rows, 4-deep ring of 40 KiB stages.
using WideTile = TileCfg<320, 256, 32, 2, 4, 4>;
// Ping-pong on 256x256 tiles: waves 0-3 (one per SIMD) own output columns
// 0-127, waves 4-7 columns 128-255; wave w and wave w + 4 share a SIMD.
using PingTile = TileCfg<256, 256, 32, 2, 4, 5, 2>;

// A wave-uniform pointer moved to scalar registers (buffer resources must be).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ void store16(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{v.x, v.y, v.z, v.w}, rsrc, off, 0, 0);
}
// The same store marked non-temporal (cache policy nt): for outputs no kernel
// of the step reads back (the weight gradients), so that their bytes do not
// push the operands still being streamed out of L2 and the last-level cache.
__device__ __forceinline__ void store16_nt(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{v.x, v.y, v.z, v.w}, rsrc, off, 0, 2);
}
__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------------------------ kernel
//
// Persistent blocks.  Block b runs on XCD b % 8 (launch indices are dealt
// round-robin over the XCDs) and takes the tiles xidx, xidx + nbx, ... of its
// XCD's contiguous share of the logical tiles, so the blocks of one XCD work
// on neighbouring tiles (an expert's weight slab and its activation rows stay
// in that XCD's L2).  With groups the real tile count is computed on the
// device from `offs` (the grid is sized without a host sync).
//
// Each block runs one continuous stream of k-steps over all its tiles: a DMA
// cursor fills the LDS ring LEAD k-steps ahead of the compute cursor (3 of 5
// stages with a block barrier every second k-step, else STAGES-1 with one per
// k-step) and runs straight across tile boundaries, so the ring never drains
// between tiles.  When the compute cursor finishes a tile, the wave writes it
// out (epilogue) while the DMA of the next tile is already in flight; the
// tile waits that follow leave that epilogue's stores outstanding, so they
// drain in the background.  Every epilogue issues the
// same number of store instructions per wave (out-of-range stores go to an
// offset past the buffer resource and are dropped), which keeps those waits
// exact.
//
// LDS layouts (per stage, per operand; 16-byte chunks, XOR-swizzled so that
// the MFMA fragment reads are free of bank conflicts: gfx950 LDS has 64 banks
// of 4 bytes, so the 16 lanes of a ds_read_b128 pass, or the 32 lanes of a
// ds_read_b64_tr_b16 pass, must touch 64 distinct banks):
//   K-contiguous operand  [R rows][BK k]:  chunk c of row r at slot c ^ kc_swizzle<BK>(r)
//   M/N-contiguous operand [BK k][R cols]: chunk c of k-row kk at slot c ^ mc_swizzle(kk)
// Each DMA instruction fills one contiguous 1 KiB block lane by lane (lane l
// -> bytes 16l..16l+15), so a lane loads whichever global chunk belongs at
// its slot.  K-contiguous fragments are one ds_read_b128; M/N-contiguous
// fragments are two ds_read_b64_tr_b16, which turn a 4 (k) x 16 (n) patch read
// by 16 lanes into 4 consecutive k per lane.

// A ds_read_b128 pass reads one chunk of 16 consecutive rows.  32-deep
// k-tiles (64-byte rows, 4 rows per 256 bytes): rows r and r + 4k differ in
// bits 2-3, which move the chunk to another 16-byte bank group.  64-deep
// k-tiles (128-byte rows, 2 rows per 256 bytes): bits 1-3 do.
template <int BK>
__device__ __forceinline__ constexpr int kc_swizzle(int r) {
  return BK == 32 ? (r >> 2) & 3 : (r >> 1) & 7;
}
// A transpose-read pass reads 32 columns (4 chunks) of 4 consecutive k-rows:
// k-row kk & 3 selects the 64-byte bank quarter (needs >= 16 chunks per k-row).
__device__ __forceinline__ constexpr int mc_swizzle(int kk) { return 4 * (kk & 3); }
// Epilogue staging of a wave's 32 x 64 bf16 pass (128-byte rows): chunk cc of
// row r at slot cc ^ stg_swizzle(r), its 8-byte halves exchanged when bit 4 of
// r is set; the 8-byte writes, the row reads and the SwiGLU gate/up reads are
// then each on distinct banks.
__device__ __forceinline__ constexpr int stg_swizzle(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

// Store instructions per wave per epilogue (all issued unconditionally).
template <int EPI, int WTM, int SM, int SN>
constexpr int epilogue_stores() {
  // bf16 outputs are staged one 32-row x 64-column pass at a time
  return EPI == EPI_F32            ? SM * SN * 4
         : EPI == EPI_SWIGLU_FWD  ? (WTM / 16) * 3 * (SN / 2)
                                  : (WTM / 8) * (SN / 2);  // EPI_BF16; EPI_WGRAD (its fp32 variant issues more)
}

template <int MODE, bool B_KCONTIG, int EPI, class CFG>
__global__ __launch_bounds__(CFG::kThreads) void grouped_gemm_kernel(const GemmParams p) {
  constexpr int BM = CFG::BM, BN = CFG::BN, BK = CFG::BK, WM = CFG::WM, WN = CFG::WN, STAGES = CFG::STAGES;
  constexpr int NWAVES = WM * WN;
  constexpr int WTM = BM / WM;  // wave tile rows
  constexpr int WTN = BN / WN;  // wave tile cols
  constexpr int SM = WTM / 32;  // 32x32 sub-tiles per wave along M
  constexpr int SN = WTN / 32;  // ... along N
  constexpr bool A_KC = (MODE == MODE_MG);
  constexpr bool B_KC = (MODE == MODE_MG) && B_KCONTIG;
  // A K-contiguous A tile occupies whole rounds of DMA instructions in LDS
  // (512 / BK rows per instruction, one instruction per wave per round): rows
  // past BM are never read and their DMA is out of range (zeros, no traffic).
  constexpr int A_ROWS = (MODE == MODE_MG) ? (BM + (512 / BK) * NWAVES - 1) / ((512 / BK) * NWAVES) * ((512 / BK) * NWAVES)
                                           : BM;
  constexpr int A_BYTES = A_ROWS * BK * 2, B_BYTES = BN * BK * 2;
  constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  constexpr int NI_A = A_BYTES / 1024, NI_B = B_BYTES / 1024;  // DMA instructions per k-tile
  // Ping-pong: the DMA of a k-tile is split by operand between the wave
  // groups (waves 0-3 fire A, waves 4-7 fire B), LPW instructions per wave.
  constexpr bool PING = CFG::PIPE == 2;
  constexpr int LPW_A = PING ? 0 : NI_A / NWAVES, LPW_B = PING ? 0 : NI_B / NWAVES;  // ... per wave and operand
  constexpr int LPW = PING ? NI_A / 4 : LPW_A + LPW_B;
  // Barrier cadence.  With a 5-deep ring the DMA runs LEAD = 3 k-steps ahead
  // and the block synchronises on even k-steps only: an even step waits for
  // its own k-tile and the next one, and the DMA of any step targets the
  // stage read three steps earlier, which every wave had left by the last
  // barrier.  Shallower rings synchronise every step with the DMA
  // STAGES - 1 steps ahead.
  //
  // The pipelined loop (CFG::PIPE) keeps the 5-deep ring with the DMA 3
  // k-steps ahead but synchronises once per k-step, in its middle: iteration
  // c reads the second half step of k-tile c, multiplies the first, waits for
  // k-tile c + 1 and synchronises, reads the first half step of c + 1 and
  // multiplies the second half of c.  Half of the DMA of k-tile c + 3 is
  // fired among each half's MFMAs.  Its stage last held k-tile c - 2, whose
  // fragments every wave had consumed (waited for) before the barrier in the
  // middle of iteration c - 1, and both halves of iteration c come after that
  // barrier.  The DMA younger than the k-tile waited for is k-tile c + 2 and
  // the first half of c + 3.
  constexpr bool PIPE = CFG::PIPE == 1;
  constexpr bool PAIR = STAGES == 5 && !PIPE && !PING;
  constexpr int LEAD = (PAIR || PIPE || PING) ? STAGES - 2 : STAGES - 1;
  // DMA younger than the k-tile waited for
  constexpr int WAIT = PING ? 2 * LPW : PIPE ? LPW + LPW / 2 : PAIR ? LPW : (STAGES - 2) * LPW;
  constexpr int RELAX = (PAIR || PIPE || PING) ? 2 : STAGES - 1;  // waits that an epilogue's stores precede
  constexpr int NST = epilogue_stores<EPI, WTM, SM, SN>();
  constexpr int SLOT = 32 * 64 * 2;  // staging bytes per wave (one 32-row x 64-column pass)
  static_assert(BK == 32 || BK == 64, "swizzles and DMA mapping cover 32- and 64-deep k-tiles");
  constexpr int RB = BK * 2;      // bytes per K-contiguous row of a k-tile
  constexpr int CPR = BK / 8;     // 16-byte chunks per K-contiguous row
  constexpr int RPI = 64 / CPR;   // K-contiguous rows per DMA instruction
  static_assert(WTM % 32 == 0 && WTN == 64, "wave tiles are whole 32x32 sub-tiles, 64 columns wide");
  static_assert(!PIPE || (STAGES == 5 && LPW % 2 == 0 && BK == 32), "the pipelined loop's stage and DMA schedule");
  // (The weight gradients keep the paired-barrier loop: on ping-pong they
  // measured 175 against 159 us (C2 down_wgrad) and 1906 against 1864 us
  // (C5 up_wgrad), the same at C4.)
  static_assert(!PING || (MODE == MODE_MG && STAGES == 5 && BK == 32 && NWAVES == 8 && WM == 2 && NI_A == NI_B &&
                          NI_A % 4 == 0),
                "the ping-pong loop's wave groups, stage and DMA schedule");
  static_assert(PING || (NI_A % NWAVES == 0 && NI_B % NWAVES == 0), "DMA instructions of each operand split evenly over waves");
  static_assert(EPI != EPI_SWIGLU_FWD || (SN % 2 == 0), "SwiGLU forward pairs gate/up sub-tiles");
  static_assert(STAGES >= 2 && STAGES <= 5, "ring depth");
  static_assert(NWAVES * SLOT <= STAGE_BYTES, "the epilogue stages every wave's pass in one ring stage");
  static_assert(WAIT + NST < 64, "vmcnt range");
  static_assert(A_KC || BM >= 128, "transpose-read swizzle needs >= 16 chunks per k-row");
  static_assert(B_KC || BN >= 128, "transpose-read swizzle needs >= 16 chunks per k-row");

  __shared__ __attribute__((aligned(1024))) char ring[STAGES * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Wave-uniform values live in scalar registers: buffer resources and the
  // DMA LDS base (M0) must be uniform.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Ping-pong wave groups: group grp = wave / 4 holds wave columns 2 grp and
  // 2 grp + 1; its four waves sit on the four SIMDs.
  const int grp = wave >> 2, w4 = wave & 3;
  const int wm = PING ? (w4 >> 1) : wave / WN, wn = PING ? grp * 2 + (w4 & 1) : wave % WN;
  const int l32 = lane & 31;
  const int khalf = lane >> 5;

  // ------------------------------------------------------ this block's tiles
  const int nbx = gridDim.x / kNumXcd;  // the grid is a multiple of kNumXcd
  const int xcd = blockIdx.x % kNumXcd, xidx = blockIdx.x / kNumXcd;
  const int real = (MODE == MODE_MG && p.offs) ? count_tiles<BM>(p.offs, p.G, p.rows, p.n_tiles) : p.total_tiles;
  int first, span;
  const int2 range = (MODE == MODE_KG && p.cost_split)
                         ? kg_cost_split<BK>(p.offs, p.G, p.rows, p.n_tiles * p.m_tiles_max, xcd)
                         : make_int2(-1, -1);
  if (range.x >= 0) {
    first = range.x;
    span = range.y - range.x;
  } else {
    const int share = (real + kNumXcd - 1) / kNumXcd;
    first = xcd * share;
    span = min(share, real - first);
  }
  // Weight gradients under skewed routing (the cost split above): the XCD's
  // tiles are dealt to its blocks in cost order, the heaviest group's first,
  // snaking (round r gives block xidx the tile at position r nbx + xidx on
  // even rounds, r nbx + nbx - 1 - xidx on odd ones), so that every block
  // gets about one tile of each cost level instead of every nbx-th tile of
  // the group-major order.  Consecutive positions are still mostly one
  // group's tiles, which the XCD's blocks take at about the same time (its
  // operand panels are shared through L2).  Lane m holds the m-th group
  // touching the range (up to 64 of them; more keep the plain deal): its
  // tiles in the range (sn_cnt, the first at sn_t0 from `first`) and the
  // tiles of the groups ranked before it (sn_pc); rank: larger k-steps
  // first, then the lower group.  Busiest block's k-steps against the mean
  // at C4's routing (simulated): up_wgrad 1.12 -> 1.09, down_wgrad 1.29 ->
  // 1.10.
  bool snake = false;
  int sn_cnt = 0, sn_t0 = 0, sn_pc = 0;
  if constexpr (MODE == MODE_KG) {
    if (range.x >= 0 && span > 0) {
      const int per_group = p.n_tiles * p.m_tiles_max;
      const int g0 = first / per_group, g1 = (first + span - 1) / per_group;
      if (g1 - g0 < kWave) {
        snake = true;
        const int g = g0 + lane;
        int cost = -1;
        if (g <= g1) {
          const int lo_t = max(first, g * per_group), hi_t = min(first + span, (g + 1) * per_group);
          sn_cnt = hi_t - lo_t;
          sn_t0 = lo_t - first;
          const int hi = min(max(p.offs[g], 0), p.rows);
          const int lo = g ? min(max(p.offs[g - 1], 0), hi) : 0;
          cost = (hi - lo + BK - 1) / BK;
        }
        int rank = 0;
        for (int m = 0; m < kWave; ++m) {
          const int cm = __builtin_amdgcn_readlane(cost, m);
          rank += (cm > cost || (cm == cost && m < lane)) ? 1 : 0;
        }
        for (int m = 0; m < kWave; ++m) {
          const int rm = __builtin_amdgcn_readlane(rank, m), cm = __builtin_amdgcn_readlane(sn_cnt, m);
          sn_pc += rm < rank ? cm : 0;
        }
      }
    }
  }
  int nt_blk;
  if (snake) {  // full rounds, plus the last partial round's slot of this block
    const int rounds = span / nbx, rem = span - rounds * nbx;
    nt_blk = rounds + (((rounds & 1) ? nbx - 1 - xidx : xidx) < rem ? 1 : 0);
  } else {
    nt_blk = span > xidx ? (span - xidx + nbx - 1) / nbx : 0;
  }
  const int ntiles = __builtin_amdgcn_readfirstlane(nt_blk);
  if (ntiles <= 0) return;

  // Lane l of a descriptor chunk describes block tile 64 * chunk + l:
  // group, first output row (absolute for MG, within the group for KG),
  // first output column, reduction rows [rb, re) (KG) or the tile's valid
  // rows end (MG), split-K index.
  struct Desc {
    int g, m0, n0, rb, re, split;
  };
  auto describe = [&](int chunk) __attribute__((always_inline)) {
    Desc d{0, 0, 0, 0, 0, 0};
    const int j = chunk * kWave + lane;
    const bool valid = j < ntiles;
    int L = first + xidx + j * nbx;
    if (MODE == MODE_KG && snake) {
      // position j nbx + slot in cost order -> the tile: the group (lane m)
      // whose positions [sn_pc, sn_pc + sn_cnt) hold it
      const int pos = j * nbx + ((j & 1) ? nbx - 1 - xidx : xidx);
      L = first;
      for (int m = 0; m < kWave; ++m) {
        const int pm = __builtin_amdgcn_readlane(sn_pc, m), cm = __builtin_amdgcn_readlane(sn_cnt, m);
        if (pos >= pm && pos < pm + cm) L = first + __builtin_amdgcn_readlane(sn_t0, m) + (pos - pm);
      }
    }
    if constexpr (MODE == MODE_MG) {
      if (p.offs) {
        // Per-lane search of the group holding tile L over the cumulative
        // per-group tile counts, one 64-group chunk at a time.
        const int target = valid ? L : 0x7fffffff;
        int found = 0, tg = 0, t0 = 0, r0 = 0, cn = 0, base = 0;
        for (int c0 = 0; c0 < p.G; c0 += kWave) {
          const int gg = c0 + lane;
          int lo = 0, hi = 0;
          if (gg < p.G) {
            hi = min(max(p.offs[gg], 0), p.rows);  // clamped: malformed offsets never address outside [0, rows)
            lo = gg ? min(max(p.offs[gg - 1], 0), hi) : 0;
          }
          const int cnt = hi - lo;
          const int nt = p.n_tiles * ((cnt + BM - 1) / BM);
          const int incl = wave_inclusive_scan(nt);
          const int tot = __builtin_amdgcn_readlane(incl, kWave - 1);
          const int t = target - base;
          int q = 0;  // smallest q with incl[q] > t
#pragma unroll
          for (int s = kWave / 2; s >= 1; s >>= 1)
            if (__shfl(incl, q + s - 1, kWave) <= t) q += s;
          const int exq = __shfl(incl - nt, q, kWave), loq = __shfl(lo, q, kWave), cq = __shfl(cnt, q, kWave);
          if (!found && t >= 0 && t < tot) {
            found = 1;
            tg = c0 + q;
            t0 = base + exq;
            r0 = loq;
            cn = cq;
          }
          base += tot;
        }
        if (valid && found) {
          const int local = L - t0;
          const int mt_g = (cn + BM - 1) / BM;
          const int nt = local / mt_g, mt = local - (local / mt_g) * mt_g;
          // The group's rows split evenly over its m-tiles (whole 32-row
          // sub-tiles): the m-tiles of one weight tile then run at the same
          // pace on neighbouring CUs and read each weight k-slice once from
          // HBM between them, where a full tile plus a short one would drift
          // apart and read it twice.  Every m-tile holds rows, since
          // (mt_g - 1) * rpt <= (mt_g - 1) * BM < cn.
          const int rpt = min(BM, ((cn + mt_g - 1) / mt_g + 31) & ~31);
          const int m0 = r0 + mt * rpt;
          d = Desc{tg, m0, nt * BN, r0, min(m0 + rpt, r0 + cn), 0};
        }
      } else {
        const int mtiles = (p.M + BM - 1) / BM;
        const int per_split = mtiles * p.n_tiles;
        const int split = L / per_split, local = L - split * per_split;
        const int nt = local / mtiles, mt = local - nt * mtiles;
        if (valid) d = Desc{0, mt * BM, nt * BN, 0, p.M, split};
      }
    } else {
      const int per_group = p.n_tiles * p.m_tiles_max;
      const int g = L / per_group, local = L - g * per_group;
      const int nt = local / p.m_tiles_max, mt = local - nt * p.m_tiles_max;
      if (valid) {
        int rb, re;
        if (p.offs) {
          re = min(max(p.offs[g], 0), p.rows);
          rb = g ? min(max(p.offs[g - 1], 0), re) : 0;
        } else {
          rb = min(g * p.chunk_rows, p.rows);
          re = min(rb + p.chunk_rows, p.rows);
        }
        d = Desc{g, mt * BM, nt * BN, rb, re, 0};
      }
    }
    return d;
  };
  auto pick = [](int v, int j) { return __builtin_amdgcn_readlane(v, j & (kWave - 1)); };

  // Per-tile scalars shared by both cursors.
  struct Tile {
    int g, m0, n0, rb, re, split, k_begin, kred, nk;
  };
  auto tile_of = [&](const Desc& d, int j) __attribute__((always_inline)) {
    Tile t;
    t.g = pick(d.g, j);
    t.m0 = pick(d.m0, j);
    t.n0 = pick(d.n0, j);
    t.rb = pick(d.rb, j);
    t.re = pick(d.re, j);
    t.split = pick(d.split, j);
    t.k_begin = (MODE == MODE_MG) ? t.split * p.k_chunk : 0;
    t.kred = (MODE == MODE_MG) ? min(p.K - t.k_begin, p.k_chunk) : (t.re - t.rb);
    t.nk = t.kred > 0 ? (t.kred + BK - 1) / BK : 0;
    return t;
  };

  // ------------------------------------------------------ DMA cursor
  // Each k-tile is NI_A + NI_B DMA instructions of 1 KiB; wave w issues A
  // instructions w*LPW_A .. w*LPW_A+LPW_A-1 (its slots j < LPW_A) and B
  // instructions w*LPW_B .. w*LPW_B+LPW_B-1 (slots j >= LPW_A).  Per lane and
  // slot: the LDS byte offset within a stage (wave-uniform), the k
  // (K-contiguous: the chunk's k; M/N-contiguous: the k-row) it adds per
  // k-tile, and a per-tile base offset (kOOB if the row or column is outside
  // the tile's valid range).
  const u32x4_t rsA = rsrc_words(p.A, p.a_bytes);
  // Row strides in bytes, in scalar registers (a ping-pong wave selects its
  // operand's at run time).
  const uint32_t lda2 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p.lda) * 2u);
  const uint32_t ldb2 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p.ldb) * 2u);
  // Slot j's operand (wave-uniform) and instruction index within the operand's k-tile.
  auto slot_is_a = [&](int j) { return PING ? grp == 0 : j < LPW_A; };
  auto slot_inst = [&](int j, bool& is_a) {
    is_a = slot_is_a(j);
    if constexpr (PING) return w4 * LPW + j;
    return is_a ? wave * LPW_A + j : wave * LPW_B + (j - LPW_A);
  };
  int dma_lds[LPW], dma_k[LPW], dma_col[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    bool is_a;
    const int li = slot_inst(j, is_a);
    dma_lds[j] = __builtin_amdgcn_readfirstlane((is_a ? 0 : A_BYTES) + li * 1024);
    dma_col[j] = 0;
    if (is_a ? A_KC : B_KC) {
      const int r = li * RPI + lane / CPR;
      dma_k[j] = ((lane % CPR) ^ kc_swizzle<BK>(r)) * 8;
    } else {
      const int cpk = (is_a ? BM : BN) / 8;  // 16-byte chunks per k-row
      dma_k[j] = li * (64 / cpk) + lane / cpk;
      dma_col[j] = ((lane % cpk) ^ mc_swizzle(dma_k[j])) * 8;  // first of the chunk's 8 columns
    }
  }

  Desc dd = describe(0);
  int dchunk = 0;
  int dj = 0, dk = 0;  // DMA cursor: block tile and k-step
  Tile dt;
  u32x4_t rsB = rsrc_words(p.B, p.b_bytes);
  // Per slot: the lane's byte offset at the tile's first k-step (kOOB if the
  // row or column lies outside the tile, or past the last tile); a k-step
  // adds a uniform amount to it.
  uint32_t dma_pre[LPW];
  // Sets the DMA cursor on block tile j (skipping tiles without k-steps);
  // past the last tile the cursor issues out-of-range loads (zeros).
  auto dma_seek = [&](int j) __attribute__((always_inline)) {
    for (;; ++j) {
      if (j >= ntiles) {
        dj = ntiles;
#pragma unroll
        for (int j2 = 0; j2 < LPW; ++j2) dma_pre[j2] = kOOB;
        return;
      }
      if ((j >> 6) != dchunk) {
        dchunk = j >> 6;
        dd = describe(dchunk);
      }
      dt = tile_of(dd, j);
      if (dt.nk > 0) break;
    }
    dj = j;
    dk = 0;
    if (MODE == MODE_MG) rsB = rsrc_words(p.B + static_cast<int64_t>(dt.g) * p.stride_bg, p.b_bytes);
    const int mc_row0 = (MODE == MODE_KG) ? dt.rb : dt.k_begin;
#pragma unroll
    for (int j2 = 0; j2 < LPW; ++j2) {
      bool is_a;
      const int li = slot_inst(j2, is_a);
      if (is_a ? A_KC : B_KC) {
        const int r = li * RPI + lane / CPR;
        const int c = (lane % CPR) ^ kc_swizzle<BK>(r);
        bool ok;
        uint32_t row_bytes;
        if (is_a) {
          const int grow = dt.m0 + r;
          ok = grow < dt.re;
          row_bytes = static_cast<uint32_t>(grow) * lda2;
        } else {
          int wrow;
          if constexpr (EPI == EPI_SWIGLU_FWD) {
            // Tile row r -> (wave column, 64-column group, half): each
            // 64-column group of a wave tile holds 32 gate rows, then the
            // 32 matching up rows, so that one 64-column epilogue pass sees
            // both halves of its act columns.
            const int wcol = r / WTN;
            const int within = r % WTN;
            const int group = within / 64;
            const int half = (within % 64) / 32;
            const int act_col = (dt.n0 / 2) + wcol * (WTN / 2) + group * 32 + (within % 32);
            ok = act_col < p.swiglu_I;
            wrow = half * p.swiglu_I + act_col;
          } else {
            wrow = dt.n0 + r;
            ok = wrow < p.N;
          }
          row_bytes = static_cast<uint32_t>(wrow) * ldb2;
        }
        dma_pre[j2] = ok ? row_bytes + static_cast<uint32_t>(c) * 16u + static_cast<uint32_t>(dt.k_begin) * 2u : kOOB;
      } else {
        const int col = (is_a ? dt.m0 : dt.n0) + dma_col[j2];
        const uint32_t ld = is_a ? lda2 : ldb2;
        dma_pre[j2] = col < (is_a ? p.M : p.N)
                          ? static_cast<uint32_t>(mc_row0 + dma_k[j2]) * ld + static_cast<uint32_t>(col) * 2u
                          : kOOB;
      }
    }
  };
  // The DMA of the cursor's next k-step into ring stage `st`, in three parts:
  // dma_prepare computes the per-lane offsets of the wave's LPW slots,
  // dma_fire(j) issues slot j, dma_advance moves the cursor.  The compute
  // loop fires the slots between its MFMA groups, so that the texture unit
  // works through the k-step's DMA while the matrix cores run instead of
  // taking every wave's burst at once.  Every k-step fires exactly LPW
  // instructions per wave.
  uint32_t doff[LPW], dlds[LPW];
  u32x4_t ra, rb;
  auto dma_prepare = [&](int st) __attribute__((always_inline)) {
    const int k0 = dk * BK;
    const int k_left = dt.kred - k0;  // k (K-contiguous) or k-rows (M/N-contiguous) left in the tile
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if constexpr (PING) {
        // every slot of a ping-pong wave is of its group's operand
        ra[w] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(grp == 0 ? rsA[w] : rsB[w]));
        rb[w] = ra[w];
      } else {
        ra[w] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(rsA[w]));
        rb[w] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(rsB[w]));
      }
    }
    const uint32_t stage_lds = lds_address(ring) + st * STAGE_BYTES;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const bool is_a = slot_is_a(j);
      const uint32_t step = (is_a ? A_KC : B_KC) ? 2u : (is_a ? lda2 : ldb2);
      // Past the last tile dma_pre is kOOB and stays out of range (the
      // added offset is below the 2 GiB operand limit).
      doff[j] = dma_k[j] < k_left ? dma_pre[j] + static_cast<uint32_t>(k0) * step : kOOB;
      dlds[j] = __builtin_amdgcn_readfirstlane(stage_lds + dma_lds[j]);
    }
  };
  auto dma_fire = [&](int j) __attribute__((always_inline)) {
    if constexpr (PING) {
      dma16(ra, doff[j], dlds[j]);
    } else {
      dma16(j < LPW_A ? ra : rb, doff[j], dlds[j]);
    }
  };
  auto dma_advance = [&]() __attribute__((always_inline)) {
    if (dj < ntiles && ++dk == dt.nk) dma_seek(dj + 1);
  };
  auto dma_issue = [&](int st) __attribute__((always_inline)) {
    dma_prepare(st);
#pragma unroll
    for (int j = 0; j < LPW; ++j) dma_fire(j);
    dma_advance();
  };

  // ------------------------------------------------------ fragment reads
  // A wave's SM row sub-tiles are interleaved with the other wave rows':
  // sub-tile i covers tile rows sub_row(i) .. +31, so that the sub-tiles of a
  // partly filled tile spread over all waves (and SIMDs).  Its SN column
  // sub-tiles are contiguous: columns wn*WTN + 32 j.
  //
  // Each lane's byte offset within a stage is precomputed per fragment class;
  // a fragment address is the stage base plus a lane offset plus a constant.
  // K-contiguous [R rows][CPR chunks]: lane reads row (tile_row + l32), chunk
  // 2 ks + khalf; fragment rows start on 32-row boundaries, so the swizzle
  // of row tile_row + l32 is that of l32.
  auto sub_row = [&](int i) { return (wm + WM * i) * 32; };
  int a_kc[BK / 16], b_kc[BK / 16];
#pragma unroll
  for (int ks = 0; ks < BK / 16; ++ks) {
    const int lane_off = l32 * RB + (((2 * ks + khalf) ^ kc_swizzle<BK>(l32)) << 4);
    a_kc[ks] = sub_row(0) * RB + lane_off;
    b_kc[ks] = A_BYTES + wn * WTN * RB + lane_off;
  }
  // M/N-contiguous [BK k-rows][R cols] (transpose reads): lane = 16 q + i reads
  // k-rows 16 ks + 8 (q/2) + 4 h + i/4 and columns tile_col + 16 (q%2) + 4 (i%4).
  // The swizzle depends only on k-row & 3 == i/4, so each 32-column sub-tile
  // has one lane offset; ks and h add constants.
  const int q16 = lane >> 4, i16 = lane & 15;
  const int tr_krow = 8 * (q16 >> 1) + (i16 >> 2);
  const int tr_col = 16 * (q16 & 1) + 4 * (i16 & 3);
  const int half8 = ((tr_col >> 2) & 1) << 3;
  int a_mc[SM], b_mc[SN];
#pragma unroll
  for (int t = 0; t < SM; ++t)
    a_mc[t] = tr_krow * BM * 2 + ((((sub_row(t) + tr_col) >> 3) ^ mc_swizzle(tr_krow)) << 4) + half8;
#pragma unroll
  for (int t = 0; t < SN; ++t)
    b_mc[t] = A_BYTES + tr_krow * BN * 2 + ((((wn * WTN + 32 * t + tr_col) >> 3) ^ mc_swizzle(tr_krow)) << 4) + half8;

  f32x16_t acc[SM][SN];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
      for (int j = 0; j < SN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  };

  // One k-tile of MFMAs over the first `na` row sub-tiles (the others hold no
  // rows of this tile; `na` is wave-uniform, so the guards are scalar
  // branches), with the prepared DMA slots fired between the MFMA groups:
  // slot s after group (ks, i) = s * (BK / 16) SM / LPW.
  auto compute = [&](int na, const char* stage) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[SM], bfr[SN];
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        if constexpr (A_KC) {
          af[i] = *reinterpret_cast<const bf16x8_t*>(stage + a_kc[ks] + i * WM * 32 * RB);
        } else {
          const char* q = stage + a_mc[i] + 16 * ks * BM * 2;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)q);
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(q + 4 * BM * 2));
          af[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      }
#pragma unroll
      for (int j = 0; j < SN; ++j) {
        if constexpr (B_KC) {
          bfr[j] = *reinterpret_cast<const bf16x8_t*>(stage + b_kc[ks] + j * 32 * RB);
        } else {
          const char* q = stage + b_mc[j] + 16 * ks * BN * 2;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)q);
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(q + 4 * BN * 2));
          bfr[j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      }
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        if (i == 0 || i < na) {
#pragma unroll
          for (int j = 0; j < SN; ++j)
            // Operands swapped: the result holds C^T fragments, so each lane
            // owns one output row and runs of 4 consecutive output columns.
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int s2 = 0; s2 < LPW; ++s2) {
          if ((s2 * (BK / 16) * SM) / LPW == ks * SM + i) {
            __builtin_amdgcn_sched_barrier(0);
            dma_fire(s2);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
  };

  // Workgroup barrier without a memory fence (a fenced barrier would drain
  // every outstanding DMA); the empty asm statements keep LDS accesses from
  // moving across it.
  auto barrier = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // ------------------------------------------------------ epilogue
  // Lane owns output row  m0 + sub_row(i) + l32  and columns
  // wcol0 + j*32 + 8*q + 4*khalf + {0..3} holding acc[i][j][4q..4q+3].
  // This wave's staging slot (no other wave touches it) in the ring stage
  // that the compute cursor has just finished: no DMA targets that stage
  // before the next block barrier, and a barrier before the epilogue
  // retires every wave's fragment reads of it.  Tiles written out before the
  // stream starts (empty weight-gradient groups) use the last stage, which
  // the prologue DMA leaves alone and no k-step fills before the first
  // barrier.
  char* slot = ring + (STAGES - 1) * STAGE_BYTES + wave * SLOT;
  auto swap_halves = [](uint4 v) { return make_uint4(v.z, v.w, v.x, v.y); };
  auto to_f32x8 = [](uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = lo_bf16(w[e]);
      f[2 * e + 1] = hi_bf16(w[e]);
    }
  };
  auto to_bf16x8 = [](const float* f) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
  };
  auto round_bf16 = [](float x) { return bf16_to_f32(f32_to_bf16(x)); };
  const __amdgpu_buffer_rsrc_t rsC2 = make_rsrc(p.C2, p.c2_bytes);  // SwiGLU pre-activation (0 bytes if absent)

  auto epilogue = [&](const Tile& t) __attribute__((always_inline)) {
    const int wcol0 = t.n0 + wn * WTN;
    const int row_limit = (MODE == MODE_MG) ? t.re : p.M;
    // Output resource: MG writes [rows, ldc]; KG one group's [M, ldc]; split-K one split's partial.
    const int esize = (EPI == EPI_F32 || (EPI == EPI_WGRAD && p.ldp)) ? 4 : 2;
    const int64_t g_off = p.bucket_rows ? static_cast<int64_t>(t.g / p.bucket_rows) * p.bucket_stride +
                                              static_cast<int64_t>(t.g % p.bucket_rows) * p.stride_cg
                                        : static_cast<int64_t>(t.g) * p.stride_cg;
    const int64_t c_base = (MODE == MODE_KG)  ? g_off
                           : (EPI == EPI_F32) ? static_cast<int64_t>(t.split) * p.split_stride
                                              : 0;
    const __amdgpu_buffer_rsrc_t rsC = make_rsrc(uniform_ptr(static_cast<char*>(p.C) + c_base * esize), p.c_bytes);
    if (EPI == EPI_F32 || (EPI == EPI_WGRAD && p.ldp)) {
      // fp32 outputs (split-K partials, fp32 weight gradients): direct 16-byte stores.
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        const int row = t.m0 + sub_row(i) + l32;
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int col = wcol0 + j * 32 + 8 * q + 4 * khalf;
            const uint32_t off = (row < row_limit && col < p.N)
                                     ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.ldc) +
                                        static_cast<uint32_t>(col)) * 4u
                                     : kOOB;
            float4 v = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
            if (EPI == EPI_WGRAD && p.accumulate) {
              const uint4 o = load16(rsC, off);
              v.x += __uint_as_float(o.x);
              v.y += __uint_as_float(o.y);
              v.z += __uint_as_float(o.z);
              v.w += __uint_as_float(o.w);
            }
            const uint4 o4 = make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                                        __float_as_uint(v.w));
            if constexpr (EPI == EPI_WGRAD) {
              store16_nt(rsC, off, o4);
            } else {
              store16(rsC, off, o4);
            }
          }
      }
      return;
    }
    // bf16 outputs go through this wave's LDS slot one 32-row pass at a time,
    // so that every store is 16 bytes per lane over whole 128-byte row segments.
    const int stg_lane = l32 * 128 + ((khalf ^ ((l32 >> 4) & 1)) << 3);
    const int stg_swz = stg_swizzle(l32);
    const int rr8 = lane >> 3, c8 = lane & 7;  // row-read lane mapping: row 8n + rr8, chunk c8
    // One pass per 32 rows (row sub-tile i) and 64 columns (column group h:
    // sub-tiles 2h and 2h + 1).
#pragma unroll
    for (int ih = 0; ih < SM * (SN / 2); ++ih) {
      const int i = ih / (SN / 2), h = ih % (SN / 2);
      const int pcol0 = wcol0 + 64 * h;     // first output column of this pass
      const int prow0 = t.m0 + sub_row(i);  // first output row of this pass
      // Output offsets of this pass's row reads and, when accumulating, the
      // existing gradient, loaded before the staging so that their latency
      // overlaps it.
      uint32_t out_off[4];
      uint4 in0[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int row = prow0 + 8 * n + rr8, col = pcol0 + c8 * 8;
        const bool ok = row < row_limit && col < p.N;
        out_off[n] = ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.ldc) + static_cast<uint32_t>(col)) * 2u
                        : kOOB;
        if constexpr (EPI == EPI_WGRAD) {
          if (p.accumulate) in0[n] = load16(rsC, out_off[n]);
        }
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int j = 2 * h + jj;
          uint2 v;
          v.x = pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
          v.y = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          *reinterpret_cast<uint2*>(slot + stg_lane + (((jj * 4 + q) ^ stg_swz) << 4)) = v;
        }
      if constexpr (EPI == EPI_SWIGLU_FWD) {
        // Slot columns 0-31 are gate, 32-63 the matching up columns.  A lane
        // takes one 8-column gate chunk and its up chunk: act = silu(gate) * up
        // with the reference's bf16 roundings (bf16 GEMM output, silu output,
        // product); gate | up go to the saved pre-activation.
        const int rr = lane >> 2, c4 = lane & 3;
        const int act_col = (t.n0 / 2) + wn * (WTN / 2) + 32 * h + c4 * 8;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int r = 16 * n + rr;
          const int swz = stg_swizzle(r);
          uint4 gv = *reinterpret_cast<const uint4*>(slot + r * 128 + ((c4 ^ swz) << 4));
          uint4 uv = *reinterpret_cast<const uint4*>(slot + r * 128 + (((c4 + 4) ^ swz) << 4));
          if (n & 1) {
            gv = swap_halves(gv);
            uv = swap_halves(uv);
          }
          const int row = prow0 + r;
          const bool ok = row < row_limit && act_col < p.swiglu_I;
          float gf[8], uf[8], af[8];
          to_f32x8(gv, gf);
          to_f32x8(uv, uf);
#pragma unroll
          for (int e = 0; e < 8; ++e) af[e] = round_bf16(silu_f(gf[e])) * uf[e];
          const uint32_t act_off = ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.ldc) +
                                         static_cast<uint32_t>(act_col)) * 2u
                                      : kOOB;
          const uint32_t pre_off = ok ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(p.ldp) +
                                         static_cast<uint32_t>(act_col)) * 2u
                                      : kOOB;
          store16(rsC, act_off, to_bf16x8(af));
          store16(rsC2, pre_off, gv);
          store16(rsC2, ok ? pre_off + static_cast<uint32_t>(p.swiglu_I) * 2u : kOOB, uv);
        }
      } else {
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const int r = 8 * n + rr8;
          uint4 v = *reinterpret_cast<const uint4*>(slot + r * 128 + ((c8 ^ stg_swizzle(r)) << 4));
          if ((n >> 1) & 1) v = swap_halves(v);
          if constexpr (EPI == EPI_BF16) {
            store16(rsC, out_off[n], v);
          } else if constexpr (EPI == EPI_WGRAD) {
            if (p.accumulate) {
              // The fp32 accumulator rounded to bf16 plus the existing bf16
              // gradient, rounded once more (torch's bf16 add of the two).
              float a[8], o[8];
              to_f32x8(v, a);
              to_f32x8(in0[n], o);
#pragma unroll
              for (int e = 0; e < 8; ++e) a[e] += o[e];
              v = to_bf16x8(a);
            }
            store16_nt(rsC, out_off[n], v);
          }
        }
      }
    }
  };

  // ------------------------------------------------------ compute cursor
  Desc cd = dd;
  int cchunk = 0;
  int cj = 0, ck = 0;
  Tile ct;
  int n_act = 0;  // row sub-tiles of this wave that hold rows of the current tile (0: no MFMAs)
  // Sets the compute cursor on block tile j.  Tiles without k-steps (empty
  // groups of a weight gradient) are written out here directly: zeros, or
  // nothing when accumulating.  Returns false past the last tile.
  int relax = 0;  // steps whose tile wait still leaves the last epilogue's stores in flight
  auto compute_seek = [&](int j) __attribute__((always_inline)) -> bool {
    for (;; ++j) {
      if (j >= ntiles) return false;
      if ((j >> 6) != cchunk) {
        cchunk = j >> 6;
        cd = describe(cchunk);
      }
      ct = tile_of(cd, j);
      zero_acc();
      if (ct.nk > 0) break;
      if constexpr (MODE == MODE_KG) {  // (MG tiles always have k-steps)
        if (!p.accumulate) {
          epilogue(ct);
          relax = RELAX;
        }
      }
    }
    cj = j;
    ck = 0;
    const int row_limit = (MODE == MODE_MG) ? ct.re : p.M;
    const int wcol0 = ct.n0 + wn * WTN;
    // Sub-tiles (and waves) whose rows or columns all lie outside the tile
    // skip the MFMAs; every wave still takes part in the DMA and the barriers.
    // Sub-tile i starts at tile row 32 (wm + WM i): i < n_act exactly when
    // it starts below the tile's last row.
    const int subs = (min(row_limit - ct.m0, BM) + 31) / 32;  // 32-row sub-tiles holding rows
    int na = subs > wm ? (subs - wm + WM - 1) / WM : 0;
    if (!(EPI == EPI_SWIGLU_FWD || wcol0 < p.N)) na = 0;
    n_act = __builtin_amdgcn_readfirstlane(min(na, SM));
    return true;
  };

  // ------------------------------------------------------ the k-step stream
  dma_seek(0);
  const bool any = compute_seek(0);
  // Stores of tiles written out above precede every DMA, so the plain tile
  // wait already covers them.
  relax = 0;
#pragma unroll
  for (int s = 0; s < LEAD; ++s) dma_issue(s);
  int cstage = 0, dstage = LEAD;
  int parity = 0;  // k-step count of the stream, mod 2
  if constexpr (PING) {
    // Ping-pong.  k-tile c of the block's stream sits in ring stage c % 5.
    // Group 0 (waves 0-3) reads k-tile c's fragments in phase 2c and
    // multiplies them in phase 2c + 1; group 1 (waves 4-7) reads them in
    // phase 2c + 1 and multiplies in phase 2c + 2.  Each phase ends with a
    // block barrier, so on every SIMD one wave issues MFMAs from registers
    // while its partner reads fragments and fires DMA.
    //
    // DMA: k-tile c's A half is fired by group 0 in phase 2c - 6 and its B
    // half by group 1 in phase 2c - 5 (the memory phases of k-tile c - 3),
    // spread among the fragment reads.  Its stage last held k-tile c - 5,
    // which group 1 read in phase 2c - 9.  Before group 0 reads k-tile c, the
    // barrier ending phase 2c - 1 follows group 0's wait for its A half (end
    // of its compute phase 2c - 1: its DMA of phases 2c - 4 and 2c - 2 may be
    // in flight) and group 1's wait for its B half (end of its memory phase
    // 2c - 1: its DMA of phases 2c - 3 and 2c - 1 may be in flight).
    //
    // A tile ending with k-tile c is written out by group 0 in phase 2c + 2
    // and by group 1 in phase 2c + 3, each staging through its half of stage
    // c % 5 (the A half for group 0, the B half for group 1), which the DMA
    // refills only from phase 2c + 4 (A) and 2c + 5 (B).
    constexpr int NR = (BK / 16) * (SM + SN);  // fragment reads per memory phase
    bf16x8_t fa[BK / 16][SM], fb[BK / 16][SN];
    auto read_frag = [&](const char* stage, int ks, int q) __attribute__((always_inline)) {
      if (q < SM) {
        const int i = q;
        if constexpr (A_KC) {
          fa[ks][i] = *reinterpret_cast<const bf16x8_t*>(stage + a_kc[ks] + i * WM * 32 * RB);
        } else {
          const char* a = stage + a_mc[i] + 16 * ks * BM * 2;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)a);
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(a + 4 * BM * 2));
          fa[ks][i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      } else {
        const int j = q - SM;
        if constexpr (B_KC) {
          fb[ks][j] = *reinterpret_cast<const bf16x8_t*>(stage + b_kc[ks] + j * 32 * RB);
        } else {
          const char* b = stage + b_mc[j] + 16 * ks * BN * 2;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)b);
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(b + 4 * BN * 2));
          fb[ks][j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      }
    };
    // This wave's half of k-tile 0 landed (its halves of k-tiles 1 and 2 are
    // younger), then every wave's, via the barrier; group 1 then waits one
    // phase.
    wait_vmcnt<WAIT>();
    barrier();
    if (grp == 1) barrier();
    bool pending = false;  // a finished tile waits for its epilogue
    int pstage = 0;        // ... and stages through this stage's half
    Tile pt = ct;
    for (;;) {
      // ---- memory phase of k-tile c (the stream's k-tile at cstage)
      if (pending) {
        pending = false;
        slot = ring + pstage * STAGE_BYTES + wave * SLOT;
        epilogue(pt);
        relax = RELAX;
        if (!compute_seek(cj + 1)) break;
      }
      const char* cur = ring + cstage * STAGE_BYTES;
      dma_prepare(dstage);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks)
#pragma unroll
        for (int q = 0; q < SM + SN; ++q) {
          read_frag(cur, ks, q);
          const int r = ks * (SM + SN) + q;
#pragma unroll
          for (int s2 = 0; s2 < LPW; ++s2)
            if (r == (s2 + 1) * NR / LPW - 1) {
              __builtin_amdgcn_sched_barrier(0);
              dma_fire(s2);
              __builtin_amdgcn_sched_barrier(0);
            }
        }
      dma_advance();
      wait_lgkmcnt0();  // the fragments are in registers before the stage can be refilled
      const bool drain = relax > 0;
      if (grp == 1) {
        if (relax > 0) --relax;
        if (drain) {
          wait_vmcnt<WAIT + NST>();
        } else {
          wait_vmcnt<WAIT>();
        }
      }
      barrier();
      // ---- compute phase of k-tile c: row sub-tiles without rows of the
      // tile skip their MFMAs (wave-uniform branches).
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks)
#pragma unroll
        for (int i = 0; i < SM; ++i)
          if (i < n_act) {
#pragma unroll
            for (int j = 0; j < SN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks][j], fa[ks][i], acc[i][j], 0, 0, 0);
          }
      if (grp == 0) {
        const bool drain0 = relax > 0;
        if (relax > 0) --relax;
        if (drain0) {
          wait_vmcnt<WAIT + NST>();
        } else {
          wait_vmcnt<WAIT>();
        }
      }
      barrier();
      const int done_stage = cstage;
      dstage = dstage + 1 == STAGES ? 0 : dstage + 1;
      cstage = cstage + 1 == STAGES ? 0 : cstage + 1;
      if (++ck == ct.nk) {
        pending = true;
        pt = ct;
        pstage = done_stage;
      }
    }
    if (grp == 0) barrier();
  } else if constexpr (PIPE) {
    // One wave per SIMD: the matrix pipe is fed only while this wave issues
    // MFMAs, so the fragments of the next half step are read into the other
    // register set while the current half step's MFMAs run, and the block
    // barrier sits where the wave has just issued a run of MFMAs.
    constexpr int HALF = LPW / 2;  // DMA instructions fired among one half step's MFMAs
    bf16x8_t fa0[SM], fb0[SN], fa1[SM], fb1[SN];
    auto read_half = [&](bf16x8_t (&fa)[SM], bf16x8_t (&fb)[SN], const char* stage, int ks)
                         __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        if constexpr (A_KC) {
          fa[i] = *reinterpret_cast<const bf16x8_t*>(stage + a_kc[ks] + i * WM * 32 * RB);
        } else {
          const char* q = stage + a_mc[i] + 16 * ks * BM * 2;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)q);
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(q + 4 * BM * 2));
          fa[i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      }
#pragma unroll
      for (int j = 0; j < SN; ++j) {
        if constexpr (B_KC) {
          fb[j] = *reinterpret_cast<const bf16x8_t*>(stage + b_kc[ks] + j * 32 * RB);
        } else {
          const char* q = stage + b_mc[j] + 16 * ks * BN * 2;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)q);
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(q + 4 * BN * 2));
          fb[j] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      }
    };
    // One half step's MFMAs over the first `na` row sub-tiles, with DMA slots
    // slot0 .. slot0 + HALF - 1 fired between the row groups.
    auto mfma_half = [&](const bf16x8_t (&fa)[SM], const bf16x8_t (&fb)[SN], int na, int slot0)
                         __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        if (i < na) {
#pragma unroll
          for (int j = 0; j < SN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int s2 = 0; s2 < HALF; ++s2) {
          if ((s2 * SM) / HALF == i) {
            __builtin_amdgcn_sched_barrier(0);
            dma_fire(slot0 + s2);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    };
    if (any) {
      // k-tile 0 landed (all but k-tiles 1 and 2 of this wave's DMA), then everyone's.
      wait_vmcnt<2 * LPW>();
      barrier();
      read_half(fa0, fb0, ring, 0);
      for (;;) {
        const char* cur = ring + cstage * STAGE_BYTES;
        const int nstage = cstage + 1 == STAGES ? 0 : cstage + 1;
        read_half(fa1, fb1, cur, 1);
        dma_prepare(dstage);
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(fa0, fb0, n_act, 0);
        // k-tile c + 1 landed: this wave's DMA (all but the WAIT younger
        // instructions, plus the last epilogue's stores while they drain),
        // then every wave's, via the barrier.
        const bool drain = relax > 0;
        if (relax > 0) --relax;
        if (drain) {
          wait_vmcnt<WAIT + NST>();
        } else {
          wait_vmcnt<WAIT>();
        }
        barrier();
        read_half(fa0, fb0, ring + nstage * STAGE_BYTES, 0);
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(fa1, fb1, n_act, HALF);
        dma_advance();
        dstage = dstage + 1 == STAGES ? 0 : dstage + 1;
        cstage = nstage;
        if (++ck == ct.nk) {
          // Stage the tile through the ring stage of its last k-tile: after
          // this barrier every wave has consumed its fragments, and the DMA
          // reaches that stage only two barriers later.
          slot = ring + (cstage == 0 ? STAGES - 1 : cstage - 1) * STAGE_BYTES + wave * SLOT;
          barrier();
          epilogue(ct);
          relax = RELAX;
          if (!compute_seek(cj + 1)) break;
        }
      }
    }
  } else if (any) {
    for (;;) {
      // k-tiles of this step (and, pairwise, the next) landed: this wave's
      // DMA (all but the WAIT younger instructions, plus the last epilogue's
      // stores while they drain), then every wave's, via the barrier; the
      // barrier also retires the reads of the stages the next DMA overwrites.
      const bool drain = relax > 0;
      if (relax > 0) --relax;
      if (!PAIR || parity == 0) {
        if (drain) {
          wait_vmcnt<WAIT + NST>();
        } else {
          wait_vmcnt<WAIT>();
        }
        barrier();
      }
      parity ^= 1;
      dma_prepare(dstage);
      if (n_act > 0) {
        // Issue priority while the wave feeds its MFMAs, so that on a shared
        // SIMD the wave with matrix work ready goes before the other wave's
        // address arithmetic and epilogue (0.4-0.6% on the expert GEMMs).
        __builtin_amdgcn_s_setprio(1);
        compute(n_act, ring + cstage * STAGE_BYTES);
        __builtin_amdgcn_s_setprio(0);
      } else {
#pragma unroll
        for (int j = 0; j < LPW; ++j) dma_fire(j);
      }
      dma_advance();
      dstage = dstage + 1 == STAGES ? 0 : dstage + 1;
      cstage = cstage + 1 == STAGES ? 0 : cstage + 1;
      if (++ck == ct.nk) {
        slot = ring + (cstage == 0 ? STAGES - 1 : cstage - 1) * STAGE_BYTES + wave * SLOT;
        barrier();
        epilogue(ct);
        relax = RELAX;
        if (!compute_seek(cj + 1)) break;
      }
    }
  }
  wait_vmcnt<0>();  // retire the trailing DMA (zeros) before the LDS is released
}

// ------------------------------------------------------------ host side

namespace {

int round_up(int x, int m) { return (x + m - 1) / m * m; }

constexpr int64_t kMaxRsrcBytes = (1ll << 31) - 64;

int set_bytes(GemmParams& p, int64_t a_bytes, int64_t b_bytes, int64_t c_bytes, const char* name) {
  MOE_REQUIRE(a_bytes < kMaxRsrcBytes && b_bytes < kMaxRsrcBytes && c_bytes < kMaxRsrcBytes, MOE_ERR_UNSUPPORTED,
              "%s: operand of %lld / %lld / %lld bytes exceeds the 2 GiB buffer-resource range", name,
              (long long)a_bytes, (long long)b_bytes, (long long)c_bytes);
  p.a_bytes = static_cast<uint32_t>(a_bytes);
  p.b_bytes = static_cast<uint32_t>(b_bytes);
  p.c_bytes = static_cast<uint32_t>(c_bytes);
  return MOE_OK;
}

template <int MODE, bool B_KCONTIG, int EPI, class CFG>
int launch(GemmParams& p, hipStream_t stream, const char* name) {
  if (p.k_splits < 1) {
    p.k_splits = 1;
    p.k_chunk = p.K;
  }
  // Output column tiles; a SwiGLU tile covers BN/2 act columns (gate + up rows).
  p.n_tiles = (EPI == EPI_SWIGLU_FWD) ? (p.swiglu_I + CFG::BN / 2 - 1) / (CFG::BN / 2)
                                      : (p.N + CFG::BN - 1) / CFG::BN;
  int64_t tiles;  // exact, or (grouped MG) the worst case; the kernel counts the real tiles itself
  if (MODE == MODE_MG) {
    p.m_tiles_max = (p.M + CFG::BM - 1) / CFG::BM + (p.offs ? p.G : 0);
    tiles = static_cast<int64_t>(p.m_tiles_max) * p.n_tiles * (p.offs ? 1 : p.k_splits);
  } else {
    p.m_tiles_max = (p.M + CFG::BM - 1) / CFG::BM;
    tiles = static_cast<int64_t>(p.G) * p.m_tiles_max * p.n_tiles;
  }
  if (tiles <= 0) return MOE_OK;
  MOE_REQUIRE(tiles < (1ll << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", name);
  if (MODE == MODE_KG) {  // cost split when every group cost and their sum fit in 30 bits
    const int64_t per_group = static_cast<int64_t>(p.n_tiles) * p.m_tiles_max;
    const int64_t bound = per_group * (p.rows / CFG::BK + p.G * (1 + kEpiSteps));
    p.cost_split = (p.offs && p.G > 1 && bound < (1ll << 30)) ? 1 : 0;
  }
  p.total_tiles = static_cast<int>(tiles);
  // Persistent grid: as many blocks as fit at once (capped by the tile
  // count), a multiple of the XCD count.
  const int dev = current_device();
  const int occ = cached_blocks_per_cu(dev, reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE, B_KCONTIG, EPI, CFG>),
                                       CFG::kThreads, 0);
  const int64_t resident = static_cast<int64_t>(device_cus(dev)) * occ / kNumXcd * kNumXcd;
  const int grid = static_cast<int>(std::max<int64_t>(kNumXcd, std::min<int64_t>(round_up(static_cast<int>(tiles),
                                                                                          kNumXcd),
                                                                                 resident)));
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE, B_KCONTIG, EPI, CFG>), dim3(grid), dim3(CFG::kThreads), 0, stream,
                     p);
  return launch_status(name);
}

// Mean rows per expert from which the forward expert GEMMs take the
// ping-pong loop (C4, 1024: the four row-grouped GEMMs 2769 against 2844 us;
// C5, 512: 5297 against 5465 us; C2, 256: up_fwd 312 against 305 us).
constexpr int64_t kPingMinMeanRows = 448;
// Mean rows per expert up to which the expert GEMMs with wide outputs take
// 320-row tiles.
constexpr int64_t kWideMaxMeanRows = 288;

// Expert GEMM over grouped rows.  256x256 tiles do the most MFMA work per
// k-step of LDS traffic, but with few output columns their grid (about one
// or two m-tiles per expert times the column tiles) ends in a poorly
// balanced last round; 384x128 tiles give one m-tile per expert of up to 384
// rows and twice the column tiles; they win when the experts hold about 256
// rows each (a training step's uniform routing).  With more rows per expert
// on average, or skewed counts, the 256x256 tile's intensity wins: the down
// projection's input gradient took 631 against 723 us at 1024 rows per
// expert (C4), 163 against 192 us at 380 rows with Zipf-skewed counts (C3).
template <bool B_KCONTIG, int EPI>
int launch_expert(GemmParams& p, hipStream_t stream, const char* name) {
  const int out_cols = (EPI == EPI_SWIGLU_FWD) ? 2 * p.swiglu_I : p.N;
  constexpr int64_t kTallMaxMeanRows = 288;
  if (out_cols <= 1024 && static_cast<int64_t>(p.rows) <= kTallMaxMeanRows * p.G)
    return launch<MODE_MG, B_KCONTIG, EPI, TallTile>(p, stream, name);
  // A training step's routing (about 256 rows per expert, a few above):
  // with 320-row tiles every expert of up to 320 rows is one m-tile, so its
  // weights stream through one CU's LDS per n-tile instead of two (C2:
  // up_fwd 280 against 318 us, down_fwd 155 against 167, up_dgrad 248
  // against 272 on ping-pong).
  if (static_cast<int64_t>(p.rows) <= kWideMaxMeanRows * p.G)
    return launch<MODE_MG, B_KCONTIG, EPI, WideTile>(p, stream, name);
  // The ping-pong loop keeps the matrix pipes fed while the partner waves
  // read fragments and fire the DMA.  It wins for the input gradients (two
  // transpose reads per weight fragment), and for the forward GEMMs once the
  // experts average several m-tiles (their weight tiles then come from L2);
  // with one or two m-tiles per expert the forward GEMMs stream every weight
  // k-slice from HBM and time the same on both loops.
  if (!B_KCONTIG || static_cast<int64_t>(p.rows) >= kPingMinMeanRows * p.G)
    return launch<MODE_MG, B_KCONTIG, EPI, PingTile>(p, stream, name);
  return launch<MODE_MG, B_KCONTIG, EPI, BigTileP>(p, stream, name);
}

// Operand checks.  `a` holds M rows, as does `b` when b_rows (the weight
// gradient's second operand); an operand of zero rows may be NULL.
int check_common(const void* a, const void* b, const int32_t* offs, int64_t G, int64_t M, int64_t N, int64_t K,
                 bool b_rows = false) {
  MOE_REQUIRE((a || M == 0) && (b || (b_rows && M == 0)), MOE_ERR_INVALID, "grouped gemm: null operand");
  MOE_REQUIRE(G >= 1 && G <= 4096, MOE_ERR_UNSUPPORTED, "grouped gemm: G=%lld outside [1,4096]", (long long)G);
  MOE_REQUIRE(offs || G == 1, MOE_ERR_INVALID, "grouped gemm: offs may be NULL only for G == 1");
  MOE_REQUIRE(M >= 0 && N > 0 && K > 0, MOE_ERR_INVALID, "grouped gemm: bad sizes M=%lld N=%lld K=%lld",
              (long long)M, (long long)N, (long long)K);
  MOE_REQUIRE(M < (1ll << 31) && N < (1 << 30) && K < (1 << 30), MOE_ERR_UNSUPPORTED, "grouped gemm: size overflow");
  MOE_REQUIRE(N % 8 == 0 && K % 8 == 0, MOE_ERR_UNSUPPORTED,
              "grouped gemm: N (%lld) and K (%lld) must be multiples of 8", (long long)N, (long long)K);
  MOE_REQUIRE(aligned16(a) && aligned16(b), MOE_ERR_INVALID, "grouped gemm: operands must be 16-byte aligned");
  return MOE_OK;
}

}  // namespace

// Router logits as split-K partials: partials[s][T][E] (f32), s < splits, each
// over the reduction range [s*k_chunk, (s+1)*k_chunk) of H.
int router_logits_partials(const bf16_t* x, const bf16_t* wr, float* partials, int T, int H, int E, int splits,
                           int k_chunk, hipStream_t stream) {
  GemmParams p{};
  p.A = x;
  p.B = wr;
  p.C = partials;
  p.G = 1;
  p.rows = p.M = T;
  p.N = E;
  p.K = H;
  p.lda = H;
  p.ldb = H;
  p.ldc = E;
  p.k_splits = splits;
  p.k_chunk = k_chunk;
  p.split_stride = static_cast<int64_t>(T) * E;
  int rc = set_bytes(p, static_cast<int64_t>(T) * H * 2, static_cast<int64_t>(E) * H * 2,
                     static_cast<int64_t>(T) * E * 4, "router logits");
  if (rc) return rc;
  return launch<MODE_MG, true, EPI_F32, SmallTile>(p, stream, "router logits (split-K)");
}

// Router weight gradient as row-chunk partials: partials[c][E][H] (f32) over
// rows [c*chunk_rows, (c+1)*chunk_rows) of T.
int router_wgrad_partials(const bf16_t* dl, const bf16_t* x, float* partials, int T, int H, int E, int chunks,
                          int chunk_rows, hipStream_t stream) {
  GemmParams p{};
  p.A = dl;
  p.B = x;
  p.C = partials;
  p.offs = nullptr;
  p.G = chunks;
  p.chunk_rows = chunk_rows;
  p.rows = T;
  p.M = E;
  p.N = H;
  p.lda = E;
  p.ldb = H;
  p.ldc = H;
  p.ldp = 1;  // f32 destination
  p.stride_cg = static_cast<int64_t>(E) * H;
  int rc = set_bytes(p, static_cast<int64_t>(T) * E * 2, static_cast<int64_t>(T) * H * 2,
                     static_cast<int64_t>(E) * H * 4, "router wgrad");
  if (rc) return rc;
  return launch<MODE_KG, false, EPI_WGRAD, SmallTile>(p, stream, "router wgrad (row chunks)");
}

// Router input gradient dx[T,H] = dl[T,E] . wr[E,H] (single group, reduction E).
int router_dgrad(const bf16_t* dl, const bf16_t* wr, bf16_t* dx, int T, int H, int E, hipStream_t stream) {
  GemmParams p{};
  p.A = dl;
  p.B = wr;
  p.C = dx;
  p.G = 1;
  p.rows = p.M = T;
  p.N = H;
  p.K = E;
  p.lda = E;
  p.ldb = H;
  p.ldc = H;
  int rc = set_bytes(p, static_cast<int64_t>(T) * E * 2, static_cast<int64_t>(E) * H * 2,
                     static_cast<int64_t>(T) * H * 2, "router dgrad");
  if (rc) return rc;
  return launch<MODE_MG, false, EPI_BF16, SmallTile>(p, stream, "router dgrad");
}

// SwiGLU backward, elementwise and in place over d_pre [rows, 2I]: the up
// half holds d_act (the bf16 input-gradient GEMM output) on entry; on exit
// d_pre = (d_gate | d_up) with the reference's bf16 roundings:
//   d_up = d * silu(gate),  d_silu = d * up,  d_gate = d_silu * s (1 + gate (1 - s)).
// One lane per 8 columns (16-byte loads and stores).  Only the rows of the
// groups, [0, offs[G-1]), are touched (read on the device, no host sync): the
// sentinel tail past them holds no pre-activations and stays as it is.
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(bf16_t* __restrict__ d_pre, const bf16_t* __restrict__ pre,
                                                         const int32_t* __restrict__ offs, int G, unsigned rows,
                                                         unsigned I) {
  const unsigned cpr = I / 8;  // 8-column chunks per half row
  const unsigned valid = offs ? static_cast<unsigned>(min(max(offs[G - 1], 0), static_cast<int>(rows))) : rows;
  const unsigned total = valid * cpr;
  for (unsigned c = blockIdx.x * blockDim.x + threadIdx.x; c < total; c += gridDim.x * blockDim.x) {
    const unsigned r = c / cpr, k = (c - r * cpr) * 8;
    bf16_t* dr = d_pre + static_cast<size_t>(r) * 2 * I;
    const bf16_t* pr = pre + static_cast<size_t>(r) * 2 * I;
    const uint4 dv = ntload16(dr + I + k);  // the last reads of d_act and of the saved pre-activations
    const uint4 gv = ntload16(pr + k);
    const uint4 uv = ntload16(pr + I + k);
    const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t og[4], ou[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float dg2[2], du2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float d = h ? hi_bf16(dw[e]) : lo_bf16(dw[e]);
        const float g = h ? hi_bf16(gw[e]) : lo_bf16(gw[e]);
        const float u = h ? hi_bf16(uw[e]) : lo_bf16(uw[e]);
        const float sg = sigmoid_f(g);
        du2[h] = d * bf16_to_f32(f32_to_bf16(g * sg));
        dg2[h] = bf16_to_f32(f32_to_bf16(d * u)) * sg * (1.0f + g * (1.0f - sg));
      }
      og[e] = pack_bf16x2(dg2[0], dg2[1]);
      ou[e] = pack_bf16x2(du2[0], du2[1]);
    }
    *reinterpret_cast<uint4*>(dr + k) = make_uint4(og[0], og[1], og[2], og[3]);
    *reinterpret_cast<uint4*>(dr + I + k) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
  }
}

}  // namespace moe

using namespace moe;

extern "C" int moe_grouped_gemm_swiglu_fwd(const void* xp, const void* w_gate_up, const int32_t* offs, int64_t G,
                                           int64_t M, int64_t H, int64_t I, void* act, void* pre, void* stream) {
  int rc = check_common(xp, w_gate_up, offs, G, M, 2 * I, H);
  if (rc) return rc;
  if (M == 0) return MOE_OK;  // no rows: empty outputs may be NULL
  MOE_REQUIRE(act && aligned16(act) && (!pre || aligned16(pre)), MOE_ERR_INVALID, "swiglu fwd: bad output pointer");
  GemmParams p{};
  p.A = static_cast<const bf16_t*>(xp);
  p.B = static_cast<const bf16_t*>(w_gate_up);
  p.C = act;
  p.C2 = pre;
  p.offs = offs;
  p.G = static_cast<int>(G);
  p.rows = p.M = static_cast<int>(M);
  p.N = static_cast<int>(2 * I);
  p.K = static_cast<int>(H);
  p.lda = H;
  p.ldb = H;
  p.ldc = I;
  p.ldp = 2 * I;
  p.stride_bg = 2 * I * H;
  p.swiglu_I = static_cast<int>(I);
  if ((rc = set_bytes(p, M * H * 2, 2 * I * H * 2, M * I * 2, "moe_grouped_gemm_swiglu_fwd"))) return rc;
  p.c2_bytes = pre ? static_cast<uint32_t>(M * 2 * I * 2) : 0u;  // < a_bytes-range: checked below
  MOE_REQUIRE(M * 2 * I * 2 < kMaxRsrcBytes, MOE_ERR_UNSUPPORTED, "swiglu fwd: pre-activation exceeds 2 GiB");
  return launch_expert<true, EPI_SWIGLU_FWD>(p, as_stream(stream), "moe_grouped_gemm_swiglu_fwd");
}

extern "C" int moe_grouped_gemm_fwd(const void* a, const void* w, const int32_t* offs, int64_t G, int64_t M, int64_t N,
                                    int64_t K, void* c, void* stream) {
  int rc = check_common(a, w, offs, G, M, N, K);
  if (rc) return rc;
  if (M == 0) return MOE_OK;
  MOE_REQUIRE(c && aligned16(c), MOE_ERR_INVALID, "grouped gemm fwd: bad output pointer");
  GemmParams p{};
  p.A = static_cast<const bf16_t*>(a);
  p.B = static_cast<const bf16_t*>(w);
  p.C = c;
  p.offs = offs;
  p.G = static_cast<int>(G);
  p.rows = p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.lda = K;
  p.ldb = K;
  p.ldc = N;
  p.stride_bg = N * K;
  if ((rc = set_bytes(p, M * K * 2, N * K * 2, M * N * 2, "moe_grouped_gemm_fwd"))) return rc;
  return launch_expert<true, EPI_BF16>(p, as_stream(stream), "moe_grouped_gemm_fwd");
}

// Router logits: f32 output, single group, no split.
extern "C" int moe_router_logits_fwd(const void* x, const void* wr, float* logits, int64_t T, int64_t H, int64_t E,
                                     void* stream) {
  int rc = check_common(x, wr, nullptr, 1, T, E, H);
  if (rc) return rc;
  if (T == 0) return MOE_OK;
  MOE_REQUIRE(logits && aligned16(logits), MOE_ERR_INVALID, "router logits: bad output pointer");
  return router_logits_partials(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), logits,
                                static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), 1,
                                static_cast<int>(H), as_stream(stream));
}

extern "C" int moe_grouped_gemm_dgrad(const void* dc, const void* w, const int32_t* offs, int64_t G, int64_t M,
                                      int64_t N, int64_t K, void* da, void* stream) {
  // da[M,K] = dc[M,N] . w[g] (w [G,N,K]): GEMM-internal reduction over N, output width K.
  int rc = check_common(dc, w, offs, G, M, K, N);
  if (rc) return rc;
  if (M == 0) return MOE_OK;
  MOE_REQUIRE(da && aligned16(da), MOE_ERR_INVALID, "grouped gemm dgrad: bad output pointer");
  GemmParams p{};
  p.A = static_cast<const bf16_t*>(dc);
  p.B = static_cast<const bf16_t*>(w);
  p.C = da;
  p.offs = offs;
  p.G = static_cast<int>(G);
  p.rows = p.M = static_cast<int>(M);
  p.N = static_cast<int>(K);
  p.K = static_cast<int>(N);
  p.lda = N;
  p.ldb = K;
  p.ldc = K;
  p.stride_bg = N * K;
  if ((rc = set_bytes(p, M * N * 2, N * K * 2, M * K * 2, "moe_grouped_gemm_dgrad"))) return rc;
  return launch_expert<false, EPI_BF16>(p, as_stream(stream), "moe_grouped_gemm_dgrad");
}

extern "C" int moe_grouped_gemm_dgrad_swiglu_bwd(const void* dy, const void* w_down, const void* pre,
                                                 const int32_t* offs, int64_t G, int64_t M, int64_t H, int64_t I,
                                                 void* d_pre, void* stream) {
  // d_act[M,I] = dy[M,H] . w_down[g] (w_down [G,H,I]) into the up half of
  // d_pre, then the SwiGLU backward in place.
  int rc = check_common(dy, w_down, offs, G, M, I, H);
  if (rc) return rc;
  if (M == 0) return MOE_OK;
  MOE_REQUIRE(pre && d_pre && aligned16(pre) && aligned16(d_pre), MOE_ERR_INVALID,
              "dgrad swiglu: bad pre/d_pre pointer");
  MOE_REQUIRE(M * I / 8 < (1ll << 31), MOE_ERR_UNSUPPORTED, "dgrad swiglu: too many rows");
  GemmParams p{};
  p.A = static_cast<const bf16_t*>(dy);
  p.B = static_cast<const bf16_t*>(w_down);
  p.C = static_cast<bf16_t*>(d_pre) + I;
  p.offs = offs;
  p.G = static_cast<int>(G);
  p.rows = p.M = static_cast<int>(M);
  p.N = static_cast<int>(I);
  p.K = static_cast<int>(H);
  p.lda = H;
  p.ldb = I;
  p.ldc = 2 * I;
  p.stride_bg = H * I;
  if ((rc = set_bytes(p, M * H * 2, H * I * 2, (M * 2 * I - I) * 2, "moe_grouped_gemm_dgrad_swiglu_bwd"))) return rc;
  hipStream_t st = as_stream(stream);
  if ((rc = launch_expert<false, EPI_BF16>(p, st, "moe_grouped_gemm_dgrad_swiglu_bwd"))) return rc;
  const int64_t chunks = M * I / 8;
  const int grid = static_cast<int>(std::min<int64_t>((chunks + 255) / 256, 4096));
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(grid), dim3(256), 0, st, static_cast<bf16_t*>(d_pre),
                     static_cast<const bf16_t*>(pre), offs, static_cast<int>(G), static_cast<unsigned>(M),
                     static_cast<unsigned>(I));
  return launch_status("moe_grouped_gemm_dgrad_swiglu_bwd (swiglu)");
}

namespace {
int wgrad(const void* dc, const void* a, const int32_t* offs, int64_t G, int64_t M, int64_t N, int64_t K, void* dw,
          int dw_is_f32, int accumulate, int64_t bucket_rows, int64_t bucket_stride, void* stream, const char* name) {
  // dw[g][N,K] = dc[rows g, N]^T . a[rows g, K]: GEMM-internal output N x K, reduction over rows.
  // With no rows at all dW is still written (zeros) or left as it is (accumulate).
  int rc = check_common(dc, a, offs, G, M, N, K, /*b_rows=*/true);
  if (rc) return rc;
  MOE_REQUIRE(dw && aligned16(dw), MOE_ERR_INVALID, "%s: bad output pointer", name);
  if (M == 0) dc = a = dw;  // zero-byte operand resources: never read, but on a valid base
  GemmParams p{};
  p.A = static_cast<const bf16_t*>(dc);
  p.B = static_cast<const bf16_t*>(a);
  p.C = dw;
  p.offs = offs;
  p.G = static_cast<int>(G);
  p.rows = static_cast<int>(M);
  p.M = static_cast<int>(N);
  p.N = static_cast<int>(K);
  p.K = 0;
  p.lda = N;
  p.ldb = K;
  p.ldc = K;
  p.ldp = dw_is_f32 ? 1 : 0;
  p.stride_cg = N * K;
  p.accumulate = accumulate ? 1 : 0;
  p.chunk_rows = static_cast<int>(M);
  p.bucket_rows = static_cast<int>(bucket_rows);
  p.bucket_stride = bucket_stride;
  if ((rc = set_bytes(p, M * N * 2, M * K * 2, N * K * (dw_is_f32 ? 4 : 2), name))) return rc;
  return launch<MODE_KG, false, EPI_WGRAD, BigTile>(p, as_stream(stream), name);
}
}  // namespace

extern "C" int moe_grouped_gemm_wgrad(const void* dc, const void* a, const int32_t* offs, int64_t G, int64_t M,
                                      int64_t N, int64_t K, void* dw, int dw_is_f32, int accumulate, void* stream) {
  return wgrad(dc, a, offs, G, M, N, K, dw, dw_is_f32, accumulate, 0, 0, stream, "moe_grouped_gemm_wgrad");
}

extern "C" int moe_grouped_gemm_wgrad_bucket(const void* dc, const void* a, const int32_t* offs, int64_t G, int64_t M,
                                             int64_t N, int64_t K, void* bucket, int64_t bucket_rows,
                                             int64_t bucket_stride, int dw_is_f32, int accumulate, void* stream) {
  const char* name = "moe_grouped_gemm_wgrad_bucket";
  MOE_REQUIRE(bucket_rows >= 1 && bucket_rows <= G, MOE_ERR_INVALID, "%s: bucket_rows=%lld outside [1, G=%lld]", name,
              (long long)bucket_rows, (long long)G);
  MOE_REQUIRE(bucket_stride >= bucket_rows * N * K, MOE_ERR_INVALID,
              "%s: bucket_stride=%lld smaller than one rank's %lld x %lld x %lld shard", name,
              (long long)bucket_stride, (long long)bucket_rows, (long long)N, (long long)K);
  MOE_REQUIRE((bucket_stride * (dw_is_f32 ? 4 : 2)) % 16 == 0, MOE_ERR_UNSUPPORTED,
              "%s: rank chunks of %lld elements are not 16-byte aligned", name, (long long)bucket_stride);
  return wgrad(dc, a, offs, G, M, N, K, bucket, dw_is_f32, accumulate, bucket_rows, bucket_stride, stream, name);
}
