// Shared device helpers for the gfx950 MoE kernels: bf16 conversion, vector
// types, wave reductions, status plumbing for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/moe_mi355x.h"

namespace moe {

constexpr int kWave = 64;  // CDNA wavefront width

typedef uint16_t bf16_t;  // raw bfloat16 bits
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Four bf16 values of a ds_read_b64_tr_b16 transpose read, and its LDS pointer type.
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// A 16-byte load marked non-temporal (cache policy nt), for the last read of
// a tensor in the step by a kernel that reads each byte once: the caches then
// keep what later kernels still read.
typedef unsigned ntv4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ntload16(const void* p) {
  const ntv4_t v = __builtin_nontemporal_load(reinterpret_cast<const ntv4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even float -> bf16 (NaN stays NaN), the rounding torch
// uses; gfx950 converts in hardware (v_cvt_pk_bf16_f32, two values at once).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Wave-wide reductions over 64 lanes with DPP lane movement (register-level,
// no LDS round trip): quad xor-1, quad xor-2, half-row mirror, row mirror,
// then row_bcast15 / row_bcast31 fold rows 0-1 and 2-3 into row 3; lane 63
// holds the result, which readlane makes wave-uniform.
namespace dpp {
constexpr int kQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141;
constexpr int kMirror = 0x140;
constexpr int kBcast15 = 0x142;   // lane 15 of row r -> row r+1 (rows 1, 3 enabled)
constexpr int kBcast31 = 0x143;   // lane 31 -> rows 2, 3
constexpr int kRowShr1 = 0x111;   // row_shr:n = 0x110 + n, within 16-lane rows
constexpr int kRowShr2 = 0x112;
constexpr int kRowShr4 = 0x114;
constexpr int kRowShr8 = 0x118;
}  // namespace dpp

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_move(float old, float src) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_move_i(int old, int src) {
  return __builtin_amdgcn_update_dpp(old, src, CTRL, ROW_MASK, 0xF, false);
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<dpp::kQuadXor1>(0.0f, v);
  v += dpp_move<dpp::kQuadXor2>(0.0f, v);
  v += dpp_move<dpp::kHalfMirror>(0.0f, v);
  v += dpp_move<dpp::kMirror>(0.0f, v);
  v += dpp_move<dpp::kBcast15, 0xA>(0.0f, v);
  v += dpp_move<dpp::kBcast31, 0xC>(0.0f, v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<dpp::kQuadXor1>(v, v));
  v = fmaxf(v, dpp_move<dpp::kQuadXor2>(v, v));
  v = fmaxf(v, dpp_move<dpp::kHalfMirror>(v, v));
  v = fmaxf(v, dpp_move<dpp::kMirror>(v, v));
  v = fmaxf(v, dpp_move<dpp::kBcast15, 0xA>(v, v));
  v = fmaxf(v, dpp_move<dpp::kBcast31, 0xC>(v, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave arg-max of (value, index): larger value wins, ties go to the lower
// index.  Lanes outside a row mask keep their own pair (old == self).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
  float ov = dpp_move<CTRL, ROW_MASK>(v, v);
  int oi = dpp_move_i<CTRL, ROW_MASK>(i, i);
  // Bitwise, not short-circuit: the compiler would otherwise branch on each
  // comparison (exec-mask save/restore around every step).
  const bool take = (ov > v) | ((ov == v) & (oi < i));
  v = take ? ov : v;
  i = take ? oi : i;
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  argmax_step<dpp::kQuadXor1>(v, i);
  argmax_step<dpp::kQuadXor2>(v, i);
  argmax_step<dpp::kHalfMirror>(v, i);
  argmax_step<dpp::kMirror>(v, i);
  argmax_step<dpp::kBcast15, 0xA>(v, i);
  argmax_step<dpp::kBcast31, 0xC>(v, i);
  v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  i = __builtin_amdgcn_readlane(i, 63);
}

// Inclusive prefix sum across the wave (every lane active): Hillis-Steele
// within each 16-lane row by DPP row shifts (lanes shifted in from outside
// the row add 0), then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15) and lane 31's into rows 2 and 3 (row_bcast:31).  DPP moves
// take a few cycles each, against an LDS round trip per step for
// ds_bpermute shuffles.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += dpp_move_i<dpp::kRowShr1>(0, v);
  v += dpp_move_i<dpp::kRowShr2>(0, v);
  v += dpp_move_i<dpp::kRowShr4>(0, v);
  v += dpp_move_i<dpp::kRowShr8>(0, v);
  v += dpp_move_i<dpp::kBcast15, 0xA>(0, v);
  v += dpp_move_i<dpp::kBcast31, 0xC>(0, v);
  return v;
}

// Thread-local error message for the C ABI.
void set_error(const char* fmt, ...);
int launch_status(const char* what);

// Per-device launch facts (mutex-guarded, computed once per device).
int current_device();
int device_cus(int dev);
// Resident blocks per CU of `kernel` (a __global__ function's address) with
// `threads` threads and `lds_bytes` of dynamic LDS, on device `dev`.
int cached_blocks_per_cu(int dev, const void* kernel, int threads, int lds_bytes);

// moe_permute_fwd's argument checks and launches, with a caller-chosen
// histogram workspace of at least moe_permute_workspace_bytes(T * k,
// num_buckets) bytes (permute.hip).
int permute_fwd_run(const void* hidden, int64_t T, int64_t H, const int64_t* ids, int64_t k, int64_t divisor,
                    int64_t num_buckets, void* permuted, int32_t* perm, int32_t* pos_of_slot, int32_t* counts,
                    int32_t* offsets, void* workspace, size_t workspace_bytes, void* stream);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kMaxSlots = 16;  // top-k slots per token handled by the k-way kernels

// A token's slots, read once per wave into wave-uniform registers: the row
// position (0 for a slot without a row, whose loads are then discarded), the
// live flag and the routing weight.  KT > 0 fixes the slot count at compile
// time; KT == 0 takes k <= kMaxSlots at run time.
template <int KT>
struct Slots {
  static constexpr int KM = KT ? KT : kMaxSlots;
  int pos[KM];
  bool ok[KM];
  float w[KM];
  __device__ __forceinline__ void load(const int32_t* pos_of_slot, const float* scores, int64_t t, int k,
                                       int n_valid) {
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      const bool live = KT ? true : j < k;
      int p = live ? pos_of_slot[t * k + j] : n_valid;
      float wj = (live && scores) ? scores[t * k + j] : 1.0f;
      p = __builtin_amdgcn_readfirstlane(p);
      wj = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, wj)));
      ok[j] = live && p < n_valid;
      pos[j] = ok[j] ? p : 0;
      w[j] = wj;
    }
  }
};

// Launches KERNEL<k> for the common top-k values (compile-time slot count)
// and KERNEL<0> (run-time k) otherwise.
#define MOE_DISPATCH_K(k, KERNEL, ...)                                      \
  switch (k) {                                                              \
    case 1: hipLaunchKernelGGL(KERNEL<1>, __VA_ARGS__); break;              \
    case 2: hipLaunchKernelGGL(KERNEL<2>, __VA_ARGS__); break;              \
    case 4: hipLaunchKernelGGL(KERNEL<4>, __VA_ARGS__); break;              \
    case 6: hipLaunchKernelGGL(KERNEL<6>, __VA_ARGS__); break;              \
    case 8: hipLaunchKernelGGL(KERNEL<8>, __VA_ARGS__); break;              \
    default: hipLaunchKernelGGL(KERNEL<0>, __VA_ARGS__); break;             \
  }

}  // namespace moe

#define MOE_REQUIRE(cond, code, ...)    \
  do {                                  \
    if (!(cond)) {                      \
      ::moe::set_error(__VA_ARGS__);    \
      return (code);                    \
    }                                   \
  } while (0)
