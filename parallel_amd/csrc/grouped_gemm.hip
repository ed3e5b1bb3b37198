// Grouped bf16 GEMMs for the MoE expert path on gfx950 (MI355X).
//
// One kernel template covers the three contraction shapes of an expert layer:
//   MG / B K-contiguous   forward      c[r,n]   = sum_k a[r,k] w[g][n,k]
//   MG / B N-contiguous   input grad   da[r,n]  = sum_k dc[r,k] w[g][k,n]
//   KG                    weight grad  dw[g][m,n] = sum_{r in g} dc[r,m] a[r,n]
// MG = groups partition the rows of the activation operand (variable M per
// expert), KG = groups partition the reduction (variable K per expert).
//
// Tiling: WM x WN waves; each wave owns a (BM/WM) x (BN/WN) block of 32x32
// MFMA sub-tiles (v_mfma_f32_32x32x16_bf16, fp32 accumulators).  The expert
// GEMMs use 256x256 tiles on 8 waves (two waves per SIMD, one workgroup per
// CU); the small router GEMMs use 128x128 on 4 waves.  Operands move from HBM
// to LDS by DMA (buffer_load_dwordx4 ... lds, no register staging) into a
// 4-deep ring of 32-deep k-tiles, so three k-tiles of loads are in flight
// while one is multiplied.  Each operand keeps its HBM layout in LDS (XOR
// swizzled): K-contiguous fragments are ds_read_b128, M/N-contiguous ones
// (weights in the input gradient, both operands of the weight gradient) are
// ds_read_b64_tr_b16 transpose reads.  Buffer loads read zero past the
// resource size, so ragged rows and the K tail need no branches.  Sub-tiles
// of a wave that lie wholly outside the valid rows/columns skip their
// fragment reads and MFMAs (the last M tile of an expert is usually short).
//
// Tiles are mapped to groups on the device from the `offs` cumsum (no host
// sync).  The logical tile order is group-major, then n-tile, then m-tile, so
// consecutive tiles share an expert's weight tile and its activation rows;
// the launch index is remapped so that each XCD (blocks are dealt round-robin
// over the 8 XCDs) gets a contiguous run of logical tiles and the sharing
// happens in that XCD's L2.
#include <type_traits>

#include "gemm.h"

namespace moe {

enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_SWIGLU_FWD = 2, EPI_SWIGLU_BWD = 3, EPI_WGRAD = 4 };
enum { MODE_MG = 0, MODE_KG = 1 };

constexpr int kNumXcd = 8;

struct GemmParams {
  const bf16_t* A;  // MG: [rows, K] (lda);  KG: [rows, M] (lda)
  const bf16_t* B;  // MG: per group (stride_bg) [N, K] or [K, N] (ldb);  KG: [rows, N] (ldb)
  void* C;          // MG: [rows, ldc];  KG: per group (stride_cg) [M, N] (ldc)
  void* C2;         // SWIGLU_FWD: pre-activation [rows, 2N] (may be null)
  const bf16_t* P;  // SWIGLU_BWD: saved pre-activation [rows, 2N]
  const int32_t* offs;
  int G;
  int rows;     // total activation rows (M for MG; sum of K for KG)
  int M, N, K;  // GEMM-internal sizes: MG: M = rows, N out cols, K reduction; KG: M x N output per group
  int64_t lda, ldb, ldc, ldp;
  int64_t stride_bg, stride_cg;
  uint32_t a_bytes;  // bytes addressable through the A buffer resource
  uint32_t b_bytes;  // bytes of one group's B (MG) or of all of B (KG)
  int swiglu_I;      // SWIGLU_FWD: intermediate size I (weight rows gate: [0,I), up: [I,2I))
  int accumulate;
  int n_tiles, m_tiles_max, total_blocks;
  int k_splits, k_chunk;  // MG without groups: split the reduction, partial outputs stacked
  int64_t split_stride;   // elements between split partials of C
  int chunk_rows;         // KG without offs and G > 1: group g = rows [g*chunk_rows, ...)
};

// ---------------------------------------------------------------- helpers

// Raw buffer loads: offsets at or past the resource's byte size read as zero
// in hardware, so out-of-range rows and the K tail need no branches.
constexpr uint32_t kOOB = 0x80000000u;  // >= every resource size (host checks < 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// Find the group g whose tile range holds logical tile L, given per-group tile
// counts ntile(g) = n_mult * ceil(cnt_g / BM).  Every wave of the block runs
// this redundantly (no LDS, no barrier).  Returns false if L is past the end.
template <int BM>
__device__ __forceinline__ bool locate_group(const int32_t* offs, int G, int rows, int n_mult, int L, int& g_out,
                                             int& tile0_out, int& row0_out, int& cnt_out) {
  const int lane = threadIdx.x & (kWave - 1);
  int base = 0;  // tiles before this chunk
  for (int c0 = 0; c0 < G; c0 += kWave) {
    int g = c0 + lane;
    int lo = 0, hi = 0;
    if (g < G) {
      // Clamped so that malformed offsets can never address rows outside [0, rows).
      hi = min(max(offs[g], 0), rows);
      lo = g ? min(max(offs[g - 1], 0), hi) : 0;
    }
    int cnt = hi - lo;
    int nt = n_mult * ((cnt + BM - 1) / BM);
    int incl = wave_inclusive_scan(nt);
    unsigned long long hit = __ballot(g < G && L < base + incl);
    if (hit) {
      // Results are wave-uniform: move them to scalar registers so the
      // compiler sees uniform control flow downstream.
      int src = __ffsll(static_cast<long long>(hit)) - 1;
      int excl = incl - nt;
      g_out = __builtin_amdgcn_readfirstlane(c0 + src);
      tile0_out = __builtin_amdgcn_readfirstlane(base + __builtin_amdgcn_readlane(excl, src));
      row0_out = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(lo, src));
      cnt_out = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(cnt, src));
      return true;
    }
    base += __builtin_amdgcn_readlane(incl, kWave - 1);
  }
  return false;
}

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

// Tile configurations: BK-deep k-tiles staged through a STAGES-deep LDS ring.
template <int BM_, int BN_, int BK_, int WM_, int WN_, int STAGES_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, STAGES = STAGES_;
  static constexpr int kThreads = 64 * WM * WN;
};
using BigTile = TileCfg<256, 256, 32, 2, 4, 4>;    // expert GEMMs: 128 KiB LDS ring, 8 waves
using SmallTile = TileCfg<128, 128, 32, 2, 2, 4>;  // router GEMMs (N = E = 128): 64 KiB ring

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Calls f(std::integral_constant<int, i>{}) for i = 0 .. N-1 (compile-time unrolled).
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// ------------------------------------------------------------------ kernel
//
// LDS layouts (per stage, per operand; 16-byte chunks, XOR-swizzled so that
// the MFMA fragment reads are free of bank conflicts: gfx950 LDS serves
// 256 bytes per clock, so the 16 lanes of a ds_read_b128 pass, or the 32
// lanes of a ds_read_b64_tr_b16 pass, must touch 64 distinct banks):
//   K-contiguous operand  [R rows][BK k]:  chunk c of row r at slot c ^ kc_swizzle(r)
//   M/N-contiguous operand [BK k][R cols]: chunk c of k-row kk at slot c ^ mc_swizzle(kk)
// Each DMA instruction (buffer_load_dwordx4 ... lds) fills one contiguous
// 1 KiB block lane by lane (lane l -> bytes 16l..16l+15), so a lane loads
// whichever global chunk belongs at its slot.  K-contiguous fragments are one
// ds_read_b128; M/N-contiguous fragments are two ds_read_b64_tr_b16, which
// turn a 4 (k) x 16 (n) patch read by 16 lanes into 4 consecutive k per lane.

// A ds_read_b128 pass reads one chunk of 16 consecutive rows: rows r and
// r + 4k differ in bits 2-3, which move the chunk to another 16-byte bank group.
__device__ __forceinline__ constexpr int kc_swizzle(int r) { return (r >> 2) & 3; }
// A transpose-read pass reads 32 columns (4 chunks) of 4 consecutive k-rows:
// k-row kk & 3 selects the 64-byte bank quarter (needs >= 16 chunks per k-row).
__device__ __forceinline__ constexpr int mc_swizzle(int kk) { return 4 * (kk & 3); }

template <int MODE, bool B_KCONTIG, int EPI, class CFG>
__global__ __launch_bounds__(CFG::kThreads) void grouped_gemm_kernel(const GemmParams p) {
  constexpr int BM = CFG::BM, BN = CFG::BN, BK = CFG::BK, WM = CFG::WM, WN = CFG::WN, STAGES = CFG::STAGES;
  constexpr int kThreads = CFG::kThreads;
  constexpr int NWAVES = WM * WN;
  constexpr int WTM = BM / WM;  // wave tile rows
  constexpr int WTN = BN / WN;  // wave tile cols
  constexpr int SM = WTM / 32;  // 32x32 sub-tiles per wave along M
  constexpr int SN = WTN / 32;  // ... along N
  constexpr bool A_KC = (MODE == MODE_MG);
  constexpr bool B_KC = (MODE == MODE_MG) && B_KCONTIG;
  constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
  constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  constexpr int NI_A = A_BYTES / 1024, NI_B = B_BYTES / 1024;  // DMA instructions per k-tile
  constexpr int LPW = (NI_A + NI_B) / NWAVES;                  // ... per wave
  static_assert(BK == 32, "swizzles and DMA mapping assume 32-deep k-tiles (4 chunks per K-contiguous row)");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tiles are whole 32x32 sub-tiles");
  static_assert((NI_A + NI_B) % NWAVES == 0 && NI_A % LPW == 0, "DMA instructions split evenly over waves");
  static_assert(EPI != EPI_SWIGLU_FWD || (SN % 2 == 0), "SwiGLU forward pairs gate/up sub-tiles");
  static_assert(STAGES >= 2 && STAGES <= 5, "ring depth");

  // One LDS array per ring stage: with distinct objects the compiler can tell
  // the stage being read from the stages being filled by DMA.
  __shared__ __attribute__((aligned(1024))) char smem0[STAGE_BYTES];
  __shared__ __attribute__((aligned(1024))) char smem1[STAGE_BYTES];
  __shared__ __attribute__((aligned(1024))) char smem2[STAGES > 2 ? STAGE_BYTES : 16];
  __shared__ __attribute__((aligned(1024))) char smem3[STAGES > 3 ? STAGE_BYTES : 16];
  __shared__ __attribute__((aligned(1024))) char smem4[STAGES > 4 ? STAGE_BYTES : 16];
  auto stage_ptr = [&](auto st) -> char* {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return smem0;
    else if constexpr (S == 1) return smem1;
    else if constexpr (S == 2) return smem2;
    else if constexpr (S == 3) return smem3;
    else return smem4;
  };

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Wave-uniform values live in scalar registers: buffer resources and the
  // DMA LDS base (M0) must be uniform, or the compiler waterfalls each load.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // XCD-aware remap of the launch index to a logical tile index: blocks are
  // dealt round-robin over the XCDs, so XCD x runs launch indices x, x + 8, ...;
  // it gets the x-th contiguous share of the logical tiles.  With groups the
  // grid is sized for the worst case, so the real tile count is computed here
  // from `offs` and the shares are cut from it (otherwise the XCDs holding the
  // upper end of the range would get no work).
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd, xcd_idx = bid / kNumXcd;
  int L;
  if (MODE == MODE_MG && p.offs) {
    const int real = count_tiles<BM>(p.offs, p.G, p.rows, p.n_tiles);
    const int share = (real + kNumXcd - 1) / kNumXcd;
    L = xcd * share + xcd_idx;
    if (xcd_idx >= share || L >= real) return;
  } else {
    L = xcd * (p.total_blocks / kNumXcd) + xcd_idx;  // total_blocks is a multiple of kNumXcd
  }

  // ------------------------------------------------------ tile -> work
  int g, m0, n0;               // group, first output row (within group for KG), first output col
  int row_begin, row_end;      // MG: absolute activation rows of the group; KG: reduction rows
  int split = 0, k_begin = 0;  // split-K partial index and its first reduction index
  if constexpr (MODE == MODE_MG) {
    if (p.offs) {
      int tile0, row0, cnt;
      if (!locate_group<BM>(p.offs, p.G, p.rows, p.n_tiles, L, g, tile0, row0, cnt)) return;
      int local = L - tile0;
      int mt_g = (cnt + BM - 1) / BM;
      int nt = local / mt_g;
      int mt = local - nt * mt_g;
      row_begin = row0;
      row_end = row0 + cnt;
      m0 = row0 + mt * BM;  // absolute row
      n0 = nt * BN;
    } else {
      int mtiles = (p.M + BM - 1) / BM;
      int per_split = mtiles * p.n_tiles;
      split = L / per_split;
      if (split >= p.k_splits) return;
      int local = L - split * per_split;
      g = 0;
      int nt = local / mtiles;
      int mt = local - nt * mtiles;
      row_begin = 0;
      row_end = p.M;
      m0 = mt * BM;
      n0 = nt * BN;
      k_begin = split * p.k_chunk;
    }
  } else {
    const int per_group = p.n_tiles * p.m_tiles_max;
    g = L / per_group;
    if (g >= p.G) return;
    int local = L - g * per_group;
    int nt = local / p.m_tiles_max;
    int mt = local - nt * p.m_tiles_max;
    if (p.offs) {
      row_end = min(max(p.offs[g], 0), p.rows);
      row_begin = g ? min(max(p.offs[g - 1], 0), row_end) : 0;
    } else {
      row_begin = min(g * p.chunk_rows, p.rows);
      row_end = min(row_begin + p.chunk_rows, p.rows);
    }
    m0 = mt * BM;
    n0 = nt * BN;
  }
  g = __builtin_amdgcn_readfirstlane(g);
  m0 = __builtin_amdgcn_readfirstlane(m0);
  n0 = __builtin_amdgcn_readfirstlane(n0);
  row_begin = __builtin_amdgcn_readfirstlane(row_begin);
  row_end = __builtin_amdgcn_readfirstlane(row_end);
  split = __builtin_amdgcn_readfirstlane(split);
  k_begin = __builtin_amdgcn_readfirstlane(k_begin);
  const bf16_t* Bg = (MODE == MODE_MG) ? p.B + static_cast<int64_t>(g) * p.stride_bg : p.B;

  // Reduction length for this tile.
  const int Kred = (MODE == MODE_MG) ? min(p.K - k_begin, p.k_chunk) : (row_end - row_begin);

  if constexpr (MODE == MODE_KG) {
    // Empty group: the weight gradient is zero (written below) or, when
    // accumulating, unchanged.
    if (Kred <= 0 && p.accumulate) return;
  }

  // Valid rows / columns of this wave's tile -> active 32x32 sub-tiles
  // (wave-uniform; inactive sub-tiles skip their fragment reads and MFMAs).
  // A SwiGLU tile keeps every sub-tile: gate and up halves pair up by index.
  const int row_limit = (MODE == MODE_MG) ? row_end : p.M;
  const int wrow0 = m0 + wm * WTM;
  const int wcol0 = n0 + wn * WTN;
  const int act_sm = __builtin_amdgcn_readfirstlane(min(SM, max(0, (row_limit - wrow0 + 31) / 32)));
  const int act_sn =
      __builtin_amdgcn_readfirstlane((EPI == EPI_SWIGLU_FWD) ? SN : min(SN, max(0, (p.N - wcol0 + 31) / 32)));
  // Waves with no valid output rows or columns skip the MFMAs (they still
  // take part in the DMA and the barriers).
  const bool wave_active = act_sm > 0 && act_sn > 0;

  f32x16_t acc[SM][SN];
#pragma unroll
  for (int i = 0; i < SM; ++i)
#pragma unroll
    for (int j = 0; j < SN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // ------------------------------------------------------ DMA setup
  // Wave w issues DMA instructions w*LPW .. w*LPW+LPW-1 of each k-tile; the
  // first NI_A belong to A, the rest to B (a wave's instructions never span
  // both).  Per lane and instruction: the LDS byte offset within a stage, a
  // fixed part of the global byte offset, and the k (K-contiguous: the k
  // chunk; M/N-contiguous: the k row) it adds per k-tile.
  const bool dma_a = (wave * LPW) < NI_A;  // wave-uniform
  const __amdgpu_buffer_rsrc_t rsA = make_rsrc(p.A, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rsB = make_rsrc(Bg, p.b_bytes);
  uint32_t dma_lds[LPW];   // stage-relative LDS byte offset of this wave's instruction j
  uint32_t dma_base[LPW];  // K-contiguous: row byte offset + chunk bytes (kOOB if the row is invalid);
                           // M/N-contiguous: column byte offset (kOOB if the column is invalid)
  int dma_k[LPW];          // K-contiguous: k of the chunk; M/N-contiguous: k row within the tile
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int inst = wave * LPW + j;
    const bool is_a = inst < NI_A;
    const int li = is_a ? inst : inst - NI_A;  // instruction index within the operand
    dma_lds[j] = (is_a ? 0 : A_BYTES) + li * 1024;
    const bool kc = is_a ? A_KC : B_KC;
    if (kc) {
      // 16 rows x 4 chunks: lane -> row li*16 + lane/4, slot lane%4.
      const int r = li * 16 + (lane >> 2);
      const int c = (lane & 3) ^ kc_swizzle(r);
      dma_k[j] = c * 8;
      bool ok;
      uint32_t row_bytes;
      if (is_a) {
        const int grow = m0 + r;
        ok = grow < row_end;
        row_bytes = static_cast<uint32_t>(grow) * static_cast<uint32_t>(p.lda) * 2u;
      } else {
        int wrow;
        if constexpr (EPI == EPI_SWIGLU_FWD) {
          // Tile row r -> (wave column, sub-tile, half): the first SN/2
          // sub-tiles of each wave column are gate rows, the rest the
          // matching up rows.
          const int wcol = r / WTN;
          const int within = r % WTN;
          const int sn = within / 32;
          const int half = sn / (SN / 2);
          const int act_col = (n0 / 2) + wcol * (WTN / 2) + (sn % (SN / 2)) * 32 + (within % 32);
          ok = act_col < p.swiglu_I;
          wrow = half * p.swiglu_I + act_col;
        } else {
          wrow = n0 + r;
          ok = wrow < p.N;
        }
        row_bytes = static_cast<uint32_t>(wrow) * static_cast<uint32_t>(p.ldb) * 2u;
      }
      dma_base[j] = ok ? row_bytes + static_cast<uint32_t>(c) * 16u : kOOB;
    } else {
      // k-rows of R columns: R/8 chunks per k-row, 64/(R/8) k-rows per instruction.
      const int R = is_a ? BM : BN;
      const int cpk = R / 8;
      const int kk = li * (64 / cpk) + lane / cpk;
      const int c = (lane % cpk) ^ mc_swizzle(kk);
      const int col = (is_a ? m0 : n0) + c * 8;
      const bool ok = col < (is_a ? p.M : p.N);
      dma_k[j] = kk;
      dma_base[j] = ok ? static_cast<uint32_t>(col) * 2u : kOOB;
    }
  }
  const int mc_row0 = (MODE == MODE_KG) ? row_begin : k_begin;  // global row of tile k = 0 (M/N-contiguous)
  const uint32_t mc_ld = static_cast<uint32_t>(dma_a ? p.lda : p.ldb) * 2u;

  // Issue the DMA of k-tile kt into ring stage ST.  The operand a wave loads
  // is wave-uniform: its buffer resource and offset formula are selected
  // without branches, so every wave runs the same straight-line code.
  auto issue_tile = [&](int kt, auto st) {
    const int k0 = kt * BK;
    char* stage = stage_ptr(st);
    const __amdgpu_buffer_rsrc_t rs = dma_a ? rsA : rsB;
    const bool kc = dma_a ? A_KC : B_KC;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int kk = k0 + dma_k[j];  // K-contiguous: k of the chunk; M/N-contiguous: k row
      const uint32_t kc_off = dma_base[j] + static_cast<uint32_t>(k_begin + k0) * 2u;
      const uint32_t mc_off = static_cast<uint32_t>(mc_row0 + kk) * mc_ld + dma_base[j];
      const uint32_t off = (kk < Kred && dma_base[j] != kOOB) ? (kc ? kc_off : mc_off) : kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(stage + dma_lds[j]), 16, off, 0, 0, 0);
    }
  };

  // ------------------------------------------------------ fragment reads
  // Each lane's byte offset within a stage is precomputed per fragment
  // class, so every fragment address is the stage array plus one lane
  // offset plus a constant.  Short address chains keep the per-stage alias
  // scopes that the compiler attaches to LDS accesses (it follows only a few
  // levels of address arithmetic); without them a fragment read waits for
  // every DMA in flight.
  const int l32 = lane & 31;
  const int khalf = lane >> 5;
  // K-contiguous [R rows][4 chunks]: lane reads row (tile_row + l32), chunk 2 ks + khalf.
  // Fragment rows start on 32-row boundaries, so row & 15 == l32 & 15.
  int a_kc[2], b_kc[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int lane_off = l32 * 64 + (((2 * ks + khalf) ^ kc_swizzle(l32)) << 4);
    a_kc[ks] = wm * WTM * 64 + lane_off;
    b_kc[ks] = A_BYTES + wn * WTN * 64 + lane_off;
  }
  // M/N-contiguous [BK k-rows][R cols] (transpose reads): lane = 16 q + i reads
  // k-rows 16 ks + 8 (q/2) + 4 h + i/4 and columns tile_col + 16 (q%2) + 4 (i%4).
  // The swizzle depends only on k-row & 3 == i/4, so each 32-column sub-tile
  // has one lane offset; ks and h add constants.
  static_assert(A_KC || BM >= 128, "transpose-read swizzle needs >= 16 chunks per k-row");
  static_assert(B_KC || BN >= 128, "transpose-read swizzle needs >= 16 chunks per k-row");
  const int q16 = lane >> 4, i16 = lane & 15;
  const int tr_krow = 8 * (q16 >> 1) + (i16 >> 2);
  const int tr_col = 16 * (q16 & 1) + 4 * (i16 & 3);
  const int half8 = ((tr_col >> 2) & 1) << 3;
  int a_mc[SM], b_mc[SN];
#pragma unroll
  for (int t = 0; t < SM; ++t)
    a_mc[t] = tr_krow * BM * 2 + ((((wm * WTM + 32 * t + tr_col) >> 3) ^ mc_swizzle(tr_krow)) << 4) + half8;
#pragma unroll
  for (int t = 0; t < SN; ++t)
    b_mc[t] = A_BYTES + tr_krow * BN * 2 + ((((wn * WTN + 32 * t + tr_col) >> 3) ^ mc_swizzle(tr_krow)) << 4) + half8;

  auto ld_frag_kc = [&](const char* stage, int lane_off, int row0_const) -> bf16x8_t {
    return *reinterpret_cast<const bf16x8_t*>(stage + lane_off + row0_const * 64);
  };
  // Sub-tile t (32 columns) of a wave tile with R columns per k-row.
  auto ld_frag_mc = [&](const char* stage, const int* lane_off, int R, int t, int ks) -> bf16x8_t {
    const char* p = stage + lane_off[t] + 16 * ks * R * 2;
    i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)p);
    i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 4 * R * 2));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, v);
  };

  auto compute_tile = [&](auto st) {
    const char* stage = stage_ptr(st);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[SM], bfr[SN];
#pragma unroll
      for (int i = 0; i < SM; ++i)
        af[i] = A_KC ? ld_frag_kc(stage, a_kc[ks], i * 32) : ld_frag_mc(stage, a_mc, BM, i, ks);
#pragma unroll
      for (int j = 0; j < SN; ++j)
        bfr[j] = B_KC ? ld_frag_kc(stage, b_kc[ks], j * 32) : ld_frag_mc(stage, b_mc, BN, j, ks);
#pragma unroll
      for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
          // Operands swapped: the result holds C^T fragments, so each lane
          // owns one output row and runs of 4 consecutive output columns.
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
  };

  // Workgroup barrier without a memory fence: a fenced barrier would make the
  // compiler drain every outstanding DMA (vmcnt(0)) each k-tile.  The empty
  // asm statements keep LDS accesses from moving across it; the DMA of the
  // tile about to be read is waited for explicitly with vmcnt.
  auto barrier = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // STAGES-deep ring: k-tile kt lives in stage kt % STAGES; the DMA of tile
  // kt + STAGES - 1 is issued right after the barrier that retires tile
  // kt - 1.  Every step issues exactly LPW DMA instructions per wave (past
  // the last tile they are all out of range and only write zeros to a stage
  // that is never read), so the wait for tile kt is always the same vmcnt.
  //
  // The steady-state loop runs whole groups of STAGES steps with no per-step
  // guard, so every stage index is a compile-time constant and the
  // compiler's LDS-DMA wait tracking (one alias scope per stage array) stays
  // exact across the back edge: a fragment read waits only for the DMA of
  // its own stage, which the explicit vmcnt above already retired.  Guarded
  // steps inside the loop would merge paths with different DMA histories at
  // the back edge and make the compiler drain every DMA (vmcnt(0)) before
  // each step's reads.  The last nk % STAGES steps run after the loop.
  const int nk = (Kred + BK - 1) / BK;
  auto step = [&](int kt, auto st) {
    constexpr int S = decltype(st)::value;
    wait_vmcnt<(STAGES - 2) * LPW>();
    barrier();
    issue_tile(kt + STAGES - 1, std::integral_constant<int, (S + STAGES - 1) % STAGES>{});
    if (wave_active) compute_tile(st);
  };
  if (nk > 0) {
    static_for<STAGES - 1>([&](auto i) { issue_tile(i, i); });
    int kt = 0;
    for (; kt + STAGES <= nk; kt += STAGES) static_for<STAGES>([&](auto i) { step(kt + i, i); });
    static_for<STAGES - 1>([&](auto i) {
      if (kt + i < nk) step(kt + i, i);
    });
    wait_vmcnt<0>();  // retire the trailing out-of-range DMA before the LDS is released
  }

  // ------------------------------------------------------ epilogue
  // Lane owns output row  wrow0 + i*32 + (lane & 31)  and columns
  // wcol0 + j*32 + 8*q + 4*(lane >> 5) + {0..3} holding acc[i][j][4q..4q+3].
  if (EPI == EPI_F32 || (EPI == EPI_WGRAD && p.ldp)) {
    // fp32 outputs (split-K partials, fp32 weight gradients): direct stores.
    float* base = static_cast<float*>(p.C) + (EPI == EPI_F32 ? split * p.split_stride
                                                                : static_cast<int64_t>(g) * p.stride_cg);
    const int col_lane = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < SM; ++i) {
      const int row = wrow0 + i * 32 + l32;
      if (row >= row_limit) continue;
#pragma unroll
      for (int j = 0; j < SN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = wcol0 + j * 32 + 8 * q + col_lane;
          if (col >= p.N) continue;
          float4* dst = reinterpret_cast<float4*>(base + static_cast<int64_t>(row) * p.ldc + col);
          float4 v = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          if (EPI == EPI_WGRAD && p.accumulate) {
            const float4 o = *dst;
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
          }
          *dst = v;
        }
    }
    return;
  }

  // bf16 outputs go through LDS so that every store is 16 bytes per lane and
  // each wave store instruction writes whole 128-byte row segments.  Each wave
  // rounds its [WTM][64] tile to bf16 into its own slice of the (now idle) ring
  // and reads it back row-wise; no other wave touches the slice, so only the
  // barrier that retires the ring is needed.  Staging layout (128-byte rows,
  // 8 chunks of 16 bytes): chunk cc of row r sits at slot cc ^ stg_swizzle(r),
  // and its two 8-byte halves are exchanged when bit 4 of r is set, which
  // keeps the 8-byte writes, the row reads and the SwiGLU gate/up reads each on
  // distinct banks.
  static_assert(WTN == 64, "staged epilogue rows are 64 columns");
  constexpr int REGION = WTM * WTN * 2;
  constexpr int PER_STAGE = STAGE_BYTES / REGION;
  static_assert(STAGE_BYTES % REGION == 0 && NWAVES <= PER_STAGE * STAGES, "ring too small to stage the tile");
  barrier();  // every wave has finished reading the ring (its DMA retired above)
  const int sidx = wave / PER_STAGE;
  char* region = (sidx == 0 ? smem0 : sidx == 1 ? smem1 : sidx == 2 ? smem2 : sidx == 3 ? smem3 : smem4) +
                 (wave - sidx * PER_STAGE) * REGION;
  auto stg_swizzle = [](int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); };
  {
    const int lane_off = l32 * 128 + ((khalf ^ ((l32 >> 4) & 1)) << 3);
    const int swz = stg_swizzle(l32);  // rows i*32 + l32 share bits 1-4 with l32
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
      for (int j = 0; j < SN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint2 v;
          v.x = pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
          v.y = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          *reinterpret_cast<uint2*>(region + i * 32 * 128 + lane_off + (((j * 4 + q) ^ swz) << 4)) = v;
        }
  }
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

  if constexpr (EPI == EPI_SWIGLU_FWD) {
    // Tile columns 0-31 are gate, 32-63 the matching up columns.  A lane takes
    // one 8-column gate chunk and its up chunk: act = silu(gate) * up with the
    // bf16 roundings of the reference (bf16 product output, silu output,
    // product), and gate | up go to the saved pre-activation.
    const int rr = lane >> 2, c4 = lane & 3;
    const int act_col = (n0 / 2) + wn * (WTN / 2) + c4 * 8;
    bf16_t* actp = static_cast<bf16_t*>(p.C);
    bf16_t* prep = static_cast<bf16_t*>(p.C2);
#pragma unroll
    for (int n = 0; n < WTM / 16; ++n) {
      const int r = 16 * n + rr;
      const int swz = stg_swizzle(r);
      uint4 gv = *reinterpret_cast<const uint4*>(region + r * 128 + ((c4 ^ swz) << 4));
      uint4 uv = *reinterpret_cast<const uint4*>(region + r * 128 + (((c4 + 4) ^ swz) << 4));
      if (n & 1) {
        gv = swap_halves(gv);
        uv = swap_halves(uv);
      }
      const int row = wrow0 + r;
      if (row < row_limit && act_col < p.swiglu_I) {
        float gf[8], uf[8], af[8];
        to_f32x8(gv, gf);
        to_f32x8(uv, uf);
#pragma unroll
        for (int e = 0; e < 8; ++e) af[e] = round_bf16(silu_f(gf[e])) * uf[e];
        *reinterpret_cast<uint4*>(actp + static_cast<int64_t>(row) * p.ldc + act_col) = to_bf16x8(af);
        if (prep) {
          bf16_t* pr = prep + static_cast<int64_t>(row) * p.ldp;
          *reinterpret_cast<uint4*>(pr + act_col) = gv;
          *reinterpret_cast<uint4*>(pr + p.swiglu_I + act_col) = uv;
        }
      }
    }
  } else {
    const int rr = lane >> 3, c8 = lane & 7;
    const int col = wcol0 + c8 * 8;
#pragma unroll
    for (int n = 0; n < WTM / 8; ++n) {
      const int r = 8 * n + rr;
      uint4 v = *reinterpret_cast<const uint4*>(region + r * 128 + ((c8 ^ stg_swizzle(r)) << 4));
      if ((n >> 1) & 1) v = swap_halves(v);
      const int row = wrow0 + r;
      if (row >= row_limit || col >= p.N) continue;
      if constexpr (EPI == EPI_BF16) {
        *reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(row) * p.ldc + col) = v;
      } else if constexpr (EPI == EPI_WGRAD) {
        uint4* dst = reinterpret_cast<uint4*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(g) * p.stride_cg +
                                              static_cast<int64_t>(row) * p.ldc + col);
        if (p.accumulate) {
          // Sum of the fp32 accumulator rounded to bf16 and the existing bf16
          // gradient, rounded once more (torch's bf16 add of the two).
          float a[8], o[8];
          to_f32x8(v, a);
          to_f32x8(*dst, o);
#pragma unroll
          for (int e = 0; e < 8; ++e) a[e] += o[e];
          v = to_bf16x8(a);
        }
        *dst = v;
      } else {  // EPI_SWIGLU_BWD: v = d_act (bf16, as the reference's bf16 product); pre = (gate | up)
        const bf16_t* pr = p.P + static_cast<int64_t>(row) * p.ldp;
        float d[8], gf[8], uf[8], dg[8], du[8];
        to_f32x8(v, d);
        to_f32x8(*reinterpret_cast<const uint4*>(pr + col), gf);
        to_f32x8(*reinterpret_cast<const uint4*>(pr + p.N + col), uf);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // act = silu(gate) * up: d_up = d * silu(gate); d_silu = d * up;
          // d_gate = d_silu * sigma (1 + gate (1 - sigma)).
          const float sg = 1.0f / (1.0f + __expf(-gf[e]));
          du[e] = d[e] * round_bf16(gf[e] * sg);
          dg[e] = round_bf16(d[e] * uf[e]) * sg * (1.0f + gf[e] * (1.0f - sg));
        }
        bf16_t* out = static_cast<bf16_t*>(p.C) + static_cast<int64_t>(row) * p.ldc;
        *reinterpret_cast<uint4*>(out + col) = to_bf16x8(dg);
        *reinterpret_cast<uint4*>(out + p.N + col) = to_bf16x8(du);
      }
    }
  }
}

// ------------------------------------------------------------ host side

namespace {

int round_up(int x, int m) { return (x + m - 1) / m * m; }

constexpr int64_t kMaxRsrcBytes = (1ll << 31) - 64;

int set_bytes(GemmParams& p, int64_t a_bytes, int64_t b_bytes, const char* name) {
  MOE_REQUIRE(a_bytes < kMaxRsrcBytes && b_bytes < kMaxRsrcBytes, MOE_ERR_UNSUPPORTED,
              "%s: operand of %lld / %lld bytes exceeds the 2 GiB buffer-resource range", name, (long long)a_bytes,
              (long long)b_bytes);
  p.a_bytes = static_cast<uint32_t>(a_bytes);
  p.b_bytes = static_cast<uint32_t>(b_bytes);
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
  int64_t blocks;
  if (MODE == MODE_MG) {
    p.m_tiles_max = (p.M + CFG::BM - 1) / CFG::BM + (p.offs ? p.G : 0);
    blocks = static_cast<int64_t>(p.m_tiles_max) * p.n_tiles * (p.offs ? 1 : p.k_splits);
  } else {
    p.m_tiles_max = (p.M + CFG::BM - 1) / CFG::BM;
    blocks = static_cast<int64_t>(p.G) * p.m_tiles_max * p.n_tiles;
  }
  if (blocks <= 0) return MOE_OK;
  MOE_REQUIRE(blocks < (1ll << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", name);
  p.total_blocks = round_up(static_cast<int>(blocks), kNumXcd);
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE, B_KCONTIG, EPI, CFG>), dim3(p.total_blocks), dim3(CFG::kThreads), 0,
                     stream, p);
  return launch_status(name);
}

int check_common(const void* a, const void* b, const int32_t* offs, int64_t G, int64_t M, int64_t N, int64_t K) {
  MOE_REQUIRE(a && b, MOE_ERR_INVALID, "grouped gemm: null operand");
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
  int rc = set_bytes(p, static_cast<int64_t>(T) * H * 2, static_cast<int64_t>(E) * H * 2, "router logits");
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
  int rc = set_bytes(p, static_cast<int64_t>(T) * E * 2, static_cast<int64_t>(T) * H * 2, "router wgrad");
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
  int rc = set_bytes(p, static_cast<int64_t>(T) * E * 2, static_cast<int64_t>(E) * H * 2, "router dgrad");
  if (rc) return rc;
  return launch<MODE_MG, false, EPI_BF16, SmallTile>(p, stream, "router dgrad");
}

}  // namespace moe

using namespace moe;

extern "C" int moe_grouped_gemm_swiglu_fwd(const void* xp, const void* w_gate_up, const int32_t* offs, int64_t G,
                                           int64_t M, int64_t H, int64_t I, void* act, void* pre, void* stream) {
  int rc = check_common(xp, w_gate_up, offs, G, M, 2 * I, H);
  if (rc) return rc;
  MOE_REQUIRE(act && aligned16(act) && (!pre || aligned16(pre)), MOE_ERR_INVALID, "swiglu fwd: bad output pointer");
  if (M == 0) return MOE_OK;
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
  if ((rc = set_bytes(p, M * H * 2, 2 * I * H * 2, "moe_grouped_gemm_swiglu_fwd"))) return rc;
  return launch<MODE_MG, true, EPI_SWIGLU_FWD, BigTile>(p, as_stream(stream), "moe_grouped_gemm_swiglu_fwd");
}

extern "C" int moe_grouped_gemm_fwd(const void* a, const void* w, const int32_t* offs, int64_t G, int64_t M, int64_t N,
                                    int64_t K, void* c, void* stream) {
  int rc = check_common(a, w, offs, G, M, N, K);
  if (rc) return rc;
  MOE_REQUIRE(c && aligned16(c), MOE_ERR_INVALID, "grouped gemm fwd: bad output pointer");
  if (M == 0) return MOE_OK;
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
  if ((rc = set_bytes(p, M * K * 2, N * K * 2, "moe_grouped_gemm_fwd"))) return rc;
  return launch<MODE_MG, true, EPI_BF16, BigTile>(p, as_stream(stream), "moe_grouped_gemm_fwd");
}

// Router logits: f32 output, single group, no split.
extern "C" int moe_router_logits_fwd(const void* x, const void* wr, float* logits, int64_t T, int64_t H, int64_t E,
                                     void* stream) {
  int rc = check_common(x, wr, nullptr, 1, T, E, H);
  if (rc) return rc;
  MOE_REQUIRE(logits && aligned16(logits), MOE_ERR_INVALID, "router logits: bad output pointer");
  if (T == 0) return MOE_OK;
  return router_logits_partials(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), logits,
                                static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), 1,
                                static_cast<int>(H), as_stream(stream));
}

extern "C" int moe_grouped_gemm_dgrad(const void* dc, const void* w, const int32_t* offs, int64_t G, int64_t M,
                                      int64_t N, int64_t K, void* da, void* stream) {
  // da[M,K] = dc[M,N] . w[g] (w [G,N,K]): GEMM-internal reduction over N, output width K.
  int rc = check_common(dc, w, offs, G, M, K, N);
  if (rc) return rc;
  MOE_REQUIRE(da && aligned16(da), MOE_ERR_INVALID, "grouped gemm dgrad: bad output pointer");
  if (M == 0) return MOE_OK;
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
  if ((rc = set_bytes(p, M * N * 2, N * K * 2, "moe_grouped_gemm_dgrad"))) return rc;
  return launch<MODE_MG, false, EPI_BF16, BigTile>(p, as_stream(stream), "moe_grouped_gemm_dgrad");
}

extern "C" int moe_grouped_gemm_dgrad_swiglu_bwd(const void* dy, const void* w_down, const void* pre,
                                                 const int32_t* offs, int64_t G, int64_t M, int64_t H, int64_t I,
                                                 void* d_pre, void* stream) {
  // d_act[M,I] = dy[M,H] . w_down[g] (w_down [G,H,I]); fused SwiGLU backward.
  int rc = check_common(dy, w_down, offs, G, M, I, H);
  if (rc) return rc;
  MOE_REQUIRE(pre && d_pre && aligned16(pre) && aligned16(d_pre), MOE_ERR_INVALID,
              "dgrad swiglu: bad pre/d_pre pointer");
  if (M == 0) return MOE_OK;
  GemmParams p{};
  p.A = static_cast<const bf16_t*>(dy);
  p.B = static_cast<const bf16_t*>(w_down);
  p.C = d_pre;
  p.P = static_cast<const bf16_t*>(pre);
  p.offs = offs;
  p.G = static_cast<int>(G);
  p.rows = p.M = static_cast<int>(M);
  p.N = static_cast<int>(I);
  p.K = static_cast<int>(H);
  p.lda = H;
  p.ldb = I;
  p.ldc = 2 * I;
  p.ldp = 2 * I;
  p.stride_bg = H * I;
  if ((rc = set_bytes(p, M * H * 2, H * I * 2, "moe_grouped_gemm_dgrad_swiglu_bwd"))) return rc;
  return launch<MODE_MG, false, EPI_SWIGLU_BWD, BigTile>(p, as_stream(stream), "moe_grouped_gemm_dgrad_swiglu_bwd");
}

extern "C" int moe_grouped_gemm_wgrad(const void* dc, const void* a, const int32_t* offs, int64_t G, int64_t M,
                                      int64_t N, int64_t K, void* dw, int dw_is_f32, int accumulate, void* stream) {
  // dw[g][N,K] = dc[rows g, N]^T . a[rows g, K]: GEMM-internal output N x K, reduction over rows.
  int rc = check_common(dc, a, offs, G, M, N, K);
  if (rc) return rc;
  MOE_REQUIRE(dw && aligned16(dw), MOE_ERR_INVALID, "grouped gemm wgrad: bad output pointer");
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
  if ((rc = set_bytes(p, M * N * 2, M * K * 2, "moe_grouped_gemm_wgrad"))) return rc;
  return launch<MODE_KG, false, EPI_WGRAD, BigTile>(p, as_stream(stream), "moe_grouped_gemm_wgrad");
}
