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
// MFMA sub-tiles (v_mfma_f32_32x32x16_bf16, fp32 accumulators in AGPRs).
// The expert GEMMs use 256x256x64 tiles on 8 waves (two waves per SIMD, one
// workgroup per CU, 144 KiB of LDS); the small router GEMMs use 128x128x64 on
// 4 waves.  Operands are staged through LDS as K-contiguous rows (row stride
// BK+8 elements) with double buffering and register prefetch of the next
// k-tile.  Operands that are contiguous along M/N in HBM are transposed in
// registers (8x8 bf16 blocks, v_perm) on their way into LDS so every MFMA
// fragment read is one 16-byte ds_read.  Global reads are raw buffer loads:
// offsets past the resource size read as zero, so ragged rows and the K tail
// need no branches.  Sub-tiles of a wave that lie wholly outside the valid
// rows/columns skip their fragment reads and MFMAs (the last M tile of an
// expert is usually short).
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

__device__ __forceinline__ uint32_t sel_lo(uint32_t a, uint32_t b) {
  // low halves: (lo16(a), lo16(b)) packed as a | b<<16
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t sel_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// Column c (0..7) of an 8x8 bf16 block given as eight 16-byte rows (row = k),
// returned as 8 bf16 (k = 0..7) in one 16-byte vector.
__device__ __forceinline__ uint4 column8(const uint4* v, int c) {
  uint32_t w[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    switch (c >> 1) {
      case 0: w[q] = v[q].x; break;
      case 1: w[q] = v[q].y; break;
      case 2: w[q] = v[q].z; break;
      default: w[q] = v[q].w; break;
    }
  }
  uint4 r;
  if (c & 1) {
    r.x = sel_hi(w[0], w[1]);
    r.y = sel_hi(w[2], w[3]);
    r.z = sel_hi(w[4], w[5]);
    r.w = sel_hi(w[6], w[7]);
  } else {
    r.x = sel_lo(w[0], w[1]);
    r.y = sel_lo(w[2], w[3]);
    r.z = sel_lo(w[4], w[5]);
    r.w = sel_lo(w[6], w[7]);
  }
  return r;
}

// Raw buffer loads: offsets at or past the resource's byte size read as zero
// in hardware, so out-of-range rows and the K tail need no branches.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;  // >= every resource size (host checks < 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(static_cast<uint32_t>(v.x), static_cast<uint32_t>(v.y), static_cast<uint32_t>(v.z),
                    static_cast<uint32_t>(v.w));
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

// Tile configurations.
template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int kThreads = 64 * WM * WN;
};
using BigTile = TileCfg<256, 256, 64, 2, 4>;    // expert GEMMs
using SmallTile = TileCfg<128, 128, 64, 2, 2>;  // router GEMMs (N = E = 128)

// ------------------------------------------------------------------ kernel

template <int MODE, bool B_KCONTIG, int EPI, class CFG>
__global__ __launch_bounds__(CFG::kThreads) void grouped_gemm_kernel(const GemmParams p) {
  constexpr int BM = CFG::BM, BN = CFG::BN, BK = CFG::BK, WM = CFG::WM, WN = CFG::WN;
  constexpr int kThreads = CFG::kThreads;
  constexpr int LDS_STRIDE = BK + 8;  // elements
  constexpr int WTM = BM / WM;        // wave tile rows
  constexpr int WTN = BN / WN;        // wave tile cols
  constexpr int SM = WTM / 32;        // 32x32 sub-tiles per wave along M
  constexpr int SN = WTN / 32;        // ... along N
  constexpr bool A_KCONTIG = (MODE == MODE_MG);
  constexpr bool BK_CONTIG = (MODE == MODE_MG) && B_KCONTIG;
  static_assert(BK % 16 == 0, "BK must be a multiple of the MFMA K (16)");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tiles are whole 32x32 sub-tiles");
  static_assert((BM * BK / 8) % kThreads == 0 && (BN * BK / 8) % kThreads == 0, "tile too small for loader");
  static_assert(EPI != EPI_SWIGLU_FWD || (SN % 2 == 0), "SwiGLU forward pairs gate/up sub-tiles");

  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BN * LDS_STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // XCD-aware remap of the launch index to a logical tile index.
  const int nb = p.total_blocks;  // multiple of kNumXcd
  const int bid = blockIdx.x;
  const int L = (bid % kNumXcd) * (nb / kNumXcd) + bid / kNumXcd;

  // ------------------------------------------------------ tile -> work
  int g, m0, n0;               // group, first output row (within group for KG), first output col
  int row_begin, row_end;      // MG: absolute activation rows of the group; KG: reduction rows
  int split = 0, k_begin = 0;  // split-K partial index and its first reduction index
  const bf16_t* Bg = p.B;
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
    Bg = p.B + static_cast<int64_t>(g) * p.stride_bg;
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
  const bool full_tile = (act_sm == SM) && (act_sn == SN);

  f32x16_t acc[SM][SN];
#pragma unroll
  for (int i = 0; i < SM; ++i)
#pragma unroll
    for (int j = 0; j < SN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // ------------------------------------------------------ loaders
  // K-contiguous operand: 16-byte chunks, chunk c -> (row c / CH, k-chunk c % CH).
  // M/N-contiguous operand: 8x8 blocks, block b -> (k-chunk b % CH, mn-block b / CH);
  // the k-chunk varies fastest across lanes, which makes each global load a
  // 128-byte run per row and the transposed 16-byte LDS stores conflict-free.
  // A transposed operand is loaded by the first half of the threads and a
  // transposed B by the second half.
  constexpr int CH = BK / 8;
  constexpr int NBA = A_KCONTIG ? 0 : CH * (BM / 8);  // 8x8 blocks of A
  constexpr int NBB = BK_CONTIG ? 0 : CH * (BN / 8);
  constexpr int A_TOFF = 0;
  constexpr int B_TOFF = BK_CONTIG ? 0 : kThreads / 2;
  constexpr int NLA = A_KCONTIG ? (BM * CH) / kThreads : (NBA + kThreads - 1) / kThreads;
  constexpr int NLB = BK_CONTIG ? (BN * CH) / kThreads : (NBB + kThreads - 1) / kThreads;
  static_assert(A_KCONTIG || NBA % kWave == 0, "A block count must be whole waves");
  static_assert(BK_CONTIG || NBB % kWave == 0, "B block count must be whole waves");

  // Buffer resources: A over all activation rows, B over this group's matrix.
  const __amdgpu_buffer_rsrc_t rsA = make_rsrc(p.A, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rsB = make_rsrc(Bg, p.b_bytes);

  // Per-thread byte offsets of K-contiguous rows (fixed over k); kOOB marks
  // rows outside the tile's valid range.
  uint32_t a_row_off[A_KCONTIG ? NLA : 1];
  uint32_t b_row_off[BK_CONTIG ? NLB : 1];

  if constexpr (A_KCONTIG) {
#pragma unroll
    for (int i = 0; i < NLA; ++i) {
      int c = tid + i * kThreads;
      int r = c / CH;
      int grow = m0 + r;
      a_row_off[i] = grow < row_end ? static_cast<uint32_t>(grow) * static_cast<uint32_t>(p.lda) * 2u : kOOB;
    }
  }
  if constexpr (BK_CONTIG) {
#pragma unroll
    for (int i = 0; i < NLB; ++i) {
      int c = tid + i * kThreads;
      int r = c / CH;
      int wrow;
      bool ok;
      if constexpr (EPI == EPI_SWIGLU_FWD) {
        // Tile row r -> (wave column, sub-tile, half): the first SN/2 sub-tiles
        // of each wave column are gate rows, the rest the matching up rows.
        int wcol = r / WTN;
        int within = r % WTN;
        int sn = within / 32;
        int half = sn / (SN / 2);
        int act_col = (n0 / 2) + wcol * (WTN / 2) + (sn % (SN / 2)) * 32 + (within % 32);
        ok = act_col < p.swiglu_I;
        wrow = half * p.swiglu_I + act_col;
      } else {
        wrow = n0 + r;
        ok = wrow < p.N;
      }
      b_row_off[i] = ok ? static_cast<uint32_t>(wrow) * static_cast<uint32_t>(p.ldb) * 2u : kOOB;
    }
  }

  uint4 ra[A_KCONTIG ? NLA : NLA * 8];
  uint4 rb[BK_CONTIG ? NLB : NLB * 8];

  auto load_tile = [&](int k0) {
    // A
    if constexpr (A_KCONTIG) {
#pragma unroll
      for (int i = 0; i < NLA; ++i) {
        int c = tid + i * kThreads;
        int kc = (c % CH) * 8;
        uint32_t off = (k0 + kc) < Kred ? a_row_off[i] + static_cast<uint32_t>(k_begin + k0 + kc) * 2u : kOOB;
        ra[i] = bload16(rsA, off);
      }
    } else {
      // A is M-contiguous: tile = BK reduction rows x BM columns, 8x8 blocks.
#pragma unroll
      for (int i = 0; i < NLA; ++i) {
        int blk = ((tid + A_TOFF) % kThreads) + i * kThreads;
        if (blk < NBA) {
          int kc = blk % CH, mb = blk / CH;
          int col = m0 + mb * 8;
          bool col_ok = col < p.M;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            int kk = k0 + kc * 8 + q;
            bool ok = col_ok && kk < Kred;
            uint32_t off = ok ? (static_cast<uint32_t>(row_begin + kk) * static_cast<uint32_t>(p.lda) +
                                 static_cast<uint32_t>(col)) * 2u
                              : kOOB;
            ra[i * 8 + q] = bload16(rsA, off);
          }
        }
      }
    }
    // B
    if constexpr (BK_CONTIG) {
#pragma unroll
      for (int i = 0; i < NLB; ++i) {
        int c = tid + i * kThreads;
        int kc = (c % CH) * 8;
        uint32_t off = (k0 + kc) < Kred ? b_row_off[i] + static_cast<uint32_t>(k_begin + k0 + kc) * 2u : kOOB;
        rb[i] = bload16(rsB, off);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NLB; ++i) {
        int blk = ((tid + B_TOFF) % kThreads) + i * kThreads;
        if (blk < NBB) {
          int kc = blk % CH, nb8 = blk / CH;
          int col = n0 + nb8 * 8;
          bool col_ok = col < p.N;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            int kk = k0 + kc * 8 + q;
            bool ok = col_ok && kk < Kred;
            int rowi = (MODE == MODE_KG) ? row_begin + kk : k_begin + kk;
            uint32_t off = ok ? (static_cast<uint32_t>(rowi) * static_cast<uint32_t>(p.ldb) +
                                 static_cast<uint32_t>(col)) * 2u
                              : kOOB;
            rb[i * 8 + q] = bload16(rsB, off);
          }
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    bf16_t* as = As[buf];
    bf16_t* bs = Bs[buf];
    if constexpr (A_KCONTIG) {
#pragma unroll
      for (int i = 0; i < NLA; ++i) {
        int c = tid + i * kThreads;
        int r = c / CH, kc = (c % CH) * 8;
        *reinterpret_cast<uint4*>(as + r * LDS_STRIDE + kc) = ra[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NLA; ++i) {
        int blk = ((tid + A_TOFF) % kThreads) + i * kThreads;
        if (blk < NBA) {
          int kc = blk % CH, mb = blk / CH;
#pragma unroll
          for (int c = 0; c < 8; ++c)
            *reinterpret_cast<uint4*>(as + (mb * 8 + c) * LDS_STRIDE + kc * 8) = column8(ra + i * 8, c);
        }
      }
    }
    if constexpr (BK_CONTIG) {
#pragma unroll
      for (int i = 0; i < NLB; ++i) {
        int c = tid + i * kThreads;
        int r = c / CH, kc = (c % CH) * 8;
        *reinterpret_cast<uint4*>(bs + r * LDS_STRIDE + kc) = rb[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NLB; ++i) {
        int blk = ((tid + B_TOFF) % kThreads) + i * kThreads;
        if (blk < NBB) {
          int kc = blk % CH, nb8 = blk / CH;
#pragma unroll
          for (int c = 0; c < 8; ++c)
            *reinterpret_cast<uint4*>(bs + (nb8 * 8 + c) * LDS_STRIDE + kc * 8) = column8(rb + i * 8, c);
        }
      }
    }
  };

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;

  // FULL: every sub-tile active, no control flow between the fragment reads
  // and the MFMAs; otherwise skip the inactive sub-tiles (uniform branches).
  auto compute_tile = [&](int buf, auto full) {
    constexpr bool FULL = decltype(full)::value;
    const bf16_t* as = As[buf] + (wm * WTM + frag_row) * LDS_STRIDE + frag_k;
    const bf16_t* bs = Bs[buf] + (wn * WTN + frag_row) * LDS_STRIDE + frag_k;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[SM], bfr[SN];
#pragma unroll
      for (int i = 0; i < SM; ++i)
        if (FULL || i < act_sm) af[i] = *reinterpret_cast<const bf16x8_t*>(as + i * 32 * LDS_STRIDE + ks * 16);
#pragma unroll
      for (int j = 0; j < SN; ++j)
        if (FULL || j < act_sn) bfr[j] = *reinterpret_cast<const bf16x8_t*>(bs + j * 32 * LDS_STRIDE + ks * 16);
#pragma unroll
      for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
          // Operands swapped: the result holds C^T fragments, so each lane
          // owns one output row and runs of 4 consecutive output columns.
          if (FULL || (i < act_sm && j < act_sn))
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
  };

  auto main_loop = [&](auto full) {
    const int nk = (Kred + BK - 1) / BK;
    if (nk <= 0) return;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tile((kt + 1) * BK);
      compute_tile(cur, full);
      if (kt + 1 < nk) store_tile(cur ^ 1);
      __syncthreads();
    }
  };
  if (full_tile)
    main_loop(std::true_type{});
  else
    main_loop(std::false_type{});

  // ------------------------------------------------------ epilogue
  // Lane owns output row  wrow0 + i*32 + (lane & 31)  and columns
  // wcol0 + j*32 + 8*q + 4*(lane >> 5) + {0..3} holding acc[i][j][4q..4q+3].
  const int col_lane = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < SM; ++i) {
    const int row = wrow0 + i * 32 + (lane & 31);
    if (row >= row_limit) continue;
    if constexpr (EPI == EPI_SWIGLU_FWD) {
#pragma unroll
      for (int j = 0; j < SN / 2; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = (n0 / 2) + wn * (WTN / 2) + j * 32 + 8 * q + col_lane;
          if (col >= p.swiglu_I) continue;
          float gt[4], up[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            gt[e] = acc[i][j][4 * q + e];
            up[e] = acc[i][j + SN / 2][4 * q + e];
          }
          uint2 act;
          act.x = pack_bf16x2(silu_f(gt[0]) * up[0], silu_f(gt[1]) * up[1]);
          act.y = pack_bf16x2(silu_f(gt[2]) * up[2], silu_f(gt[3]) * up[3]);
          *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(row) * p.ldc + col) = act;
          if (p.C2) {
            bf16_t* pre = static_cast<bf16_t*>(p.C2) + static_cast<int64_t>(row) * p.ldp;
            uint2 gv, uv;
            gv.x = pack_bf16x2(gt[0], gt[1]);
            gv.y = pack_bf16x2(gt[2], gt[3]);
            uv.x = pack_bf16x2(up[0], up[1]);
            uv.y = pack_bf16x2(up[2], up[3]);
            *reinterpret_cast<uint2*>(pre + col) = gv;
            *reinterpret_cast<uint2*>(pre + p.swiglu_I + col) = uv;
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < SN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = wcol0 + j * 32 + 8 * q + col_lane;
          if (col >= p.N) continue;
          float v0 = acc[i][j][4 * q + 0], v1 = acc[i][j][4 * q + 1];
          float v2 = acc[i][j][4 * q + 2], v3 = acc[i][j][4 * q + 3];
          if constexpr (EPI == EPI_BF16) {
            uint2 o;
            o.x = pack_bf16x2(v0, v1);
            o.y = pack_bf16x2(v2, v3);
            *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.C) + static_cast<int64_t>(row) * p.ldc + col) = o;
          } else if constexpr (EPI == EPI_F32) {
            *reinterpret_cast<float4*>(static_cast<float*>(p.C) + split * p.split_stride +
                                       static_cast<int64_t>(row) * p.ldc + col) = make_float4(v0, v1, v2, v3);
          } else if constexpr (EPI == EPI_SWIGLU_BWD) {
            // v = d_act at (row, col..col+3); pre holds (gate | up).
            const bf16_t* pre = p.P + static_cast<int64_t>(row) * p.ldp;
            uint2 gw = *reinterpret_cast<const uint2*>(pre + col);
            uint2 uw = *reinterpret_cast<const uint2*>(pre + p.N + col);
            float gt[4] = {lo_bf16(gw.x), hi_bf16(gw.x), lo_bf16(gw.y), hi_bf16(gw.y)};
            float up[4] = {lo_bf16(uw.x), hi_bf16(uw.x), lo_bf16(uw.y), hi_bf16(uw.y)};
            float da[4] = {v0, v1, v2, v3};
            float dg[4], du[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float s = 1.0f / (1.0f + __expf(-gt[e]));
              float silu = gt[e] * s;
              du[e] = da[e] * silu;
              dg[e] = da[e] * up[e] * s * (1.0f + gt[e] * (1.0f - s));
            }
            bf16_t* out = static_cast<bf16_t*>(p.C) + static_cast<int64_t>(row) * p.ldc;
            uint2 og, ou;
            og.x = pack_bf16x2(dg[0], dg[1]);
            og.y = pack_bf16x2(dg[2], dg[3]);
            ou.x = pack_bf16x2(du[0], du[1]);
            ou.y = pack_bf16x2(du[2], du[3]);
            *reinterpret_cast<uint2*>(out + col) = og;
            *reinterpret_cast<uint2*>(out + p.N + col) = ou;
          } else {  // EPI_WGRAD: bf16 or f32 destination chosen by ldp (0 = bf16, 1 = f32)
            int64_t off = static_cast<int64_t>(g) * p.stride_cg + static_cast<int64_t>(row) * p.ldc + col;
            if (p.ldp) {
              float4* dst = reinterpret_cast<float4*>(static_cast<float*>(p.C) + off);
              if (p.accumulate) {
                float4 o = *dst;
                v0 += o.x; v1 += o.y; v2 += o.z; v3 += o.w;
              }
              *dst = make_float4(v0, v1, v2, v3);
            } else {
              uint2* dst = reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.C) + off);
              if (p.accumulate) {
                uint2 o = *dst;
                v0 += lo_bf16(o.x); v1 += hi_bf16(o.x); v2 += lo_bf16(o.y); v3 += hi_bf16(o.y);
              }
              uint2 ob;
              ob.x = pack_bf16x2(v0, v1);
              ob.y = pack_bf16x2(v2, v3);
              *dst = ob;
            }
          }
        }
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
