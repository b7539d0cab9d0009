// Shared helpers for the gfx950 kernels of libcoopt_amd.so: number formats, wave-level
// reductions, and the host-side error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/coopt_amd.h"

#define COOPT_WAVE 64

// ---------------------------------------------------------------------------------------
// Host side: per-thread error text and argument checks.
// ---------------------------------------------------------------------------------------
namespace coopt {

void set_error(const std::string& msg);
void clear_error();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks hipGetLastError() after a launch; records the message on failure.
int check_launch(const char* what);

}  // namespace coopt

#define COOPT_REQUIRE(cond, msg)                                 \
  do {                                                           \
    if (!(cond)) {                                               \
      coopt::set_error(std::string(__func__) + ": " + (msg));   \
      return COOPT_EINVAL;                                       \
    }                                                            \
  } while (0)

// ---------------------------------------------------------------------------------------
// Device side: number formats.  bf16 values travel as raw uint16_t bit patterns.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16, round to nearest even (NaN stays NaN), as torch's .to(torch.bfloat16).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> fp16, round to nearest even with fp16 subnormals (v_cvt_f16_f32 in the default
// rounding mode), as torch's .to(torch.float16).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// The value lane l ^ 16 (lane l ^ 32) holds, for a symmetric combination: v_permlane16_swap
// (v_permlane32_swap) run on two copies of v leaves every lane's own value in one result and
// its partner's in the other, so op(first, second) = op(v, partner).  A VALU exchange, unlike
// __shfl_xor's ds_bpermute round trip through the LDS crossbar.
typedef unsigned int u32x2_pl_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float max_xor16(float v) {
  const u32x2_pl_t r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const u32x2_pl_t r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float v) {
  const u32x2_pl_t r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const u32x2_pl_t r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- DPP lane exchanges (VALU, no LDS round trip) -------------------------------------
// dpp_ctrl codes of GFX9: quad permutes, mirrors within a 16-lane row or 8-lane half row,
// shifts within a row, and the row broadcasts used for wave-wide scans.
namespace dpp {
constexpr int kXor1 = 0xB1;        // quad_perm [1,0,3,2]: lane i ^ 1
constexpr int kXor2 = 0x4E;        // quad_perm [2,3,0,1]: lane i ^ 2
constexpr int kRowShr1 = 0x111;    // lane i - 1 within the row
constexpr int kRowShr2 = 0x112;
constexpr int kRowShr4 = 0x114;
constexpr int kRowShr8 = 0x118;
constexpr int kRowMirror = 0x140;      // lane 15 - i within the row
constexpr int kRowHalfMirror = 0x141;  // lane 7 - i within the half row
constexpr int kRowBcast15 = 0x142;     // lane 15 of the previous row
constexpr int kRowBcast31 = 0x143;     // lane 31
constexpr int kWaveShr1 = 0x138;       // lane i - 1 across the wave
}  // namespace dpp

// v of the lane CTRL names; lanes without a source (or in rows outside ROW_MASK) get `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t old = 0) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {  // lanes without a source get +0.0
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(u));
  const uint32_t hi = dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(u >> 32));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}

// (own, partner) values of lane i ^ 16 / i ^ 32 for a double (see max_xor16 below: the pair
// comes back in lane-dependent order, the same for both halves).
__device__ __forceinline__ void swap_xor_f64(double v, bool x32, double& a, double& b) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(u), hi = static_cast<uint32_t>(u >> 32);
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  const u2 rl = x32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                    : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const u2 rh = x32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                    : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  a = __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(rh[0]) << 32) | rl[0]));
  b = __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(rh[1]) << 32) | rl[1]));
}

// Wave-wide fp64 sum.  Every step adds a lane's value to its partner's, and a + b == b + a,
// so every lane ends with the same bits.
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
  v += dpp_f64<dpp::kXor1>(v);
  v += dpp_f64<dpp::kXor2>(v);
  v += dpp_f64<dpp::kRowHalfMirror>(v);
  v += dpp_f64<dpp::kRowMirror>(v);
  double a, b;
  swap_xor_f64(v, false, a, b);
  v = a + b;
  swap_xor_f64(v, true, a, b);
  return a + b;
}

// Wave-wide fp32 minimum, every lane the same result.
__device__ __forceinline__ float wave_min_f32_dpp(float v) {
  v = fminf(v, dpp_f32<dpp::kXor1>(v));
  v = fminf(v, dpp_f32<dpp::kXor2>(v));
  v = fminf(v, dpp_f32<dpp::kRowHalfMirror>(v));
  v = fminf(v, dpp_f32<dpp::kRowMirror>(v));
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  u2 r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Wave-wide fp32 maximum, every lane the same result (DPP and permlane swaps: no LDS round
// trips, unlike a shuffle reduction).
__device__ __forceinline__ float wave_max_f32_dpp(float v) {
  v = fmaxf(v, dpp_f32<dpp::kXor1>(v));
  v = fmaxf(v, dpp_f32<dpp::kXor2>(v));
  v = fmaxf(v, dpp_f32<dpp::kRowHalfMirror>(v));
  v = fmaxf(v, dpp_f32<dpp::kRowMirror>(v));
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  u2 r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Inclusive fp64 prefix sum over the wave's lanes (lane 0 first): Hillis-Steele within each
// 16-lane row, then the row totals carried forward with the row broadcasts.  `excl` gets the
// previous lane's inclusive value (+0.0 in lane 0), bit for bit.
__device__ __forceinline__ double wave_incl_scan_f64(double v, double& excl) {
  v += dpp_f64<dpp::kRowShr1>(v);
  v += dpp_f64<dpp::kRowShr2>(v);
  v += dpp_f64<dpp::kRowShr4>(v);
  v += dpp_f64<dpp::kRowShr8>(v);
  v += dpp_f64<dpp::kRowBcast15, 0xa>(v);
  v += dpp_f64<dpp::kRowBcast31, 0xc>(v);
  excl = dpp_f64<dpp::kWaveShr1>(v);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, COOPT_WAVE);
}

// Max over aligned groups of `G` consecutive lanes (G a power of two <= 64), every lane of a
// group the same result: DPP inside a 16-lane row (quad swaps, then the half-row and row
// mirrors), permlane swaps across rows -- VALU exchanges, no LDS round trip per step.
template <int G>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G must be a power of two <= 64");
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  if constexpr (G >= 2) v = mx(v, dpp_u32<dpp::kXor1>(v));
  if constexpr (G >= 4) v = mx(v, dpp_u32<dpp::kXor2>(v));
  if constexpr (G >= 8) v = mx(v, dpp_u32<dpp::kRowHalfMirror>(v));
  if constexpr (G >= 16) v = mx(v, dpp_u32<dpp::kRowMirror>(v));
  if constexpr (G >= 32) {
    const u32x2_pl_t r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = mx(r[0], r[1]);
  }
  if constexpr (G >= 64) {
    const u32x2_pl_t r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = mx(r[0], r[1]);
  }
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int m = 1; m < COOPT_WAVE; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, COOPT_WAVE));
  return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 1; m < COOPT_WAVE; m <<= 1) v += __shfl_xor(v, m, COOPT_WAVE);
  return v;
}

// Sum of ks (<= 16) fp32 partial slices p[k * slice], k = 0..ks-1, added in order; every
// load is issued before the first add.
__device__ __forceinline__ float4 sum_partials4(const float* p, int ks, int64_t slice) {
  float4 v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k)
    if (k < ks) v[k] = *reinterpret_cast<const float4*>(p + k * slice);
  float4 s = v[0];
#pragma unroll
  for (int k = 1; k < 16; ++k)
    if (k < ks) {
      s.x += v[k].x; s.y += v[k].y; s.z += v[k].z; s.w += v[k].w;
    }
  return s;
}

// The same sum for ks <= KS (a compile-time bound): the KS loads are unconditional -- slice
// indices past ks - 1 repeat the last slice, which hits the cache -- so a caller can issue
// every load of several groups before the first add, and the compiler's wait counts stay
// exact (a load under a branch makes it wait for every load in flight).  Same order of adds
// as sum_partials4, so the same result.
template <int KS>
struct Partials4 {
  float4 v[KS];
  __device__ __forceinline__ void load(const float* p, int ks, int64_t slice) {
#pragma unroll
    for (int k = 0; k < KS; ++k)
      v[k] = *reinterpret_cast<const float4*>(p + static_cast<int64_t>(k < ks ? k : ks - 1) * slice);
  }
  __device__ __forceinline__ float4 sum(int ks) const {
    float4 s = v[0];
#pragma unroll
    for (int k = 1; k < KS; ++k)
      if (k < ks) {
        s.x += v[k].x; s.y += v[k].y; s.z += v[k].z; s.w += v[k].w;
      }
    return s;
  }
};

// Smallest power of two >= ks (ks in [1, 16]).
inline int partials_bound(int ks) {
  int b = 1;
  while (b < ks) b <<= 1;
  return b;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int m = 1; m < COOPT_WAVE; m <<= 1) v += __shfl_xor(v, m, COOPT_WAVE);
  return v;
}
