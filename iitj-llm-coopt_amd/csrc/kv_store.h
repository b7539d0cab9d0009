// Device helpers shared by the kernels that write the paged KV cache: the symmetric absmax
// INT8 quantiser, the per-chunk KV store, and neox RoPE on one 16-byte chunk of a head vector.
//
// Quantisation follows kv_tier_manager.quantize (engine/kv_tier_manager.py:21-31) as torch
// executes it on a GPU tensor:
//   amax  = max |x| over the last dim (exact in any format)
//   s32   = max(amax, fp32(1e-8)) * fp32(1/qmax)   -- torch's GPU path turns "tensor / python
//           scalar" into a multiply by the fp32 reciprocal of the scalar
//   code  = int8(clamp(round_half_even(x / s32), -qmax, qmax))   -- IEEE fp32 division
//   scale = fp16(s32), round to nearest even
#pragma once

#include "common.h"

namespace {

constexpr float kClampMin = 1e-8f;  // torch converts clamp_min(1e-8) to the tensor's fp32

template <int QMAX>
__device__ __forceinline__ float quant_scale(float amax) {
  return fmaxf(amax, kClampMin) * (1.0f / static_cast<float>(QMAX));
}

// code = rint(fl(x / s32)) clamped to [-QMAX, QMAX], fl the IEEE fp32 quotient, computed as
// rint(x * r32) with r32 = v_rcp_f32(s32) (1 ulp).  Because s32 >= amax / 127 up to rounding,
// |x / s32| < 128, where an ulp is at most 2^-17: the reciprocal's relative error (2^-23)
// and the product's rounding leave x * r32 within 2.5 ulp of x / s32, hence within 3 ulp
// (< 2^-14) of fl(x / s32), so both round to the same integer unless x * r32 lies within
// kNearTie of a half-integer.  There the IEEE division decides.
// The result is the IEEE path's for every input (ties included), at a fraction of its work.
constexpr float kNearTie = 0x1p-14f;

template <int QMAX>
__device__ __forceinline__ int quant_code(float x, float s32, float r32) {
  const float q = x * r32;
  float r = rintf(q);
  if (fabsf(q - r) >= 0.5f - kNearTie) r = rintf(x / s32);
  r = fminf(fmaxf(r, -static_cast<float>(QMAX)), static_cast<float>(QMAX));
  return static_cast<int>(r);
}

// quant_code of the 8 bf16 elements in w[0..3] (element 2i in the low half of w[i]), with one
// branch for the lane: if any element is near a boundary, all 8 take the IEEE division.
template <int QMAX>
__device__ __forceinline__ void quant_codes8(const uint32_t (&w)[4], float s32, int (&code)[8]) {
  const float r32 = __builtin_amdgcn_rcpf(s32);
  float x[8], r[8];
  bool near = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = bf16_to_f32(static_cast<uint16_t>(w[e / 2] >> (16 * (e & 1))));
    const float q = x[e] * r32;
    r[e] = rintf(q);
    near |= fabsf(q - r[e]) >= 0.5f - kNearTie;
  }
  if (near) {
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = rintf(x[e] / s32);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    code[e] = static_cast<int>(fminf(fmaxf(r[e], -static_cast<float>(QMAX)), static_cast<float>(QMAX)));
}

// quant_codes8<127> of the 8 bf16 elements in w[0..3], returned as the packed INT8 codes
// (element e in byte e % 4 of word e / 4).  The code is formed in the low byte of a float:
// for |r| <= 127, fp32(r + 1.5 * 2^23) rounds r to the nearest integer, ties to even (the
// sum lies in [2^23, 2^24), where the ulp is 1) and holds it, two's complement, in the low
// mantissa bits, so one add replaces rint, the float-to-int conversion and the masking.
// q is clamped to +-127 before rounding, which for integer bounds equals clamping the
// rounded value.  Same codes as quant_codes8<127>, ties and non-finite inputs included.
__device__ __forceinline__ uint2 quant_pack8_i8(const uint32_t (&w)[4], float s32) {
  constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
  const float r32 = __builtin_amdgcn_rcpf(s32);
  float x[8], f[8];
  bool near = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = bf16_to_f32(static_cast<uint16_t>(w[e / 2] >> (16 * (e & 1))));
    const float q = fminf(fmaxf(x[e] * r32, -127.0f), 127.0f);
    f[e] = q + kMagic;
    near |= fabsf(q - (f[e] - kMagic)) >= 0.5f - kNearTie;
  }
  if (near) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(x[e] / s32, -127.0f), 127.0f) + kMagic;
  }
  uint32_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = __float_as_uint(f[e]);
  // bytes 0 of four words: perm selects from {hi:lo} (lo bytes 0-3, hi bytes 4-7); 0x0c = 0
  const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u) |
                      __builtin_amdgcn_perm(b[3], b[2], 0x04000c0cu);
  const uint32_t hi = __builtin_amdgcn_perm(b[5], b[4], 0x0c0c0400u) |
                      __builtin_amdgcn_perm(b[7], b[6], 0x04000c0cu);
  return make_uint2(lo, hi);
}

// INT8 codes of two adjacent chunks (16 elements, words of a and b) of a vector covered by
// G2 lanes, two chunks a lane: the codes and scale quant_chunk<2 G2, 8> gives the two chunks'
// lanes, as one 16-byte word.  Every lane of the group must call it together.
struct QuantPair {
  uint4 codes;
  uint16_t scale;
};
template <int G2>
__device__ __forceinline__ QuantPair quant_pair8(const uint4& a, const uint4& b) {
  const uint32_t w0[4] = {a.x, a.y, a.z, a.w};
  const uint32_t w1[4] = {b.x, b.y, b.z, b.w};
  uint32_t amax = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    amax = max(amax, max(w0[e] & 0x7fffu, (w0[e] >> 16) & 0x7fffu));
    amax = max(amax, max(w1[e] & 0x7fffu, (w1[e] >> 16) & 0x7fffu));
  }
  amax = group_max_u32<G2>(amax);
  const float s32 = quant_scale<127>(bf16_to_f32(static_cast<uint16_t>(amax)));
  const uint2 p0 = quant_pack8_i8(w0, s32), p1 = quant_pack8_i8(w1, s32);
  return QuantPair{make_uint4(p0.x, p0.y, p1.x, p1.y), f32_to_f16(s32)};
}

// ---------------------------------------------------------------------------------------
// KV write.  One lane per 16-byte chunk (8 bf16) of a (token, head) vector; G = D/8 lanes
// (an aligned power-of-two group inside the wave) cover one vector, and each lane handles
// the same chunk of K and of V, so every load and store is a 16- or 8-byte access.
// ---------------------------------------------------------------------------------------
// Lane c of a G-lane group stores elements [8c, 8c + 8) of one (token, head) K and V vector
// at cache element offset c_off: bf16 as is, or INT8 codes with the group's fp16 scale at
// s_off (kv_tier_manager.quantize(x, 8) per vector, engine/kv_tier_manager.py:21-31).
// The K / V words are nontemporal stores (a group writes whole 128- or 256-byte rows).
// Alternated with plain stores on MI355X: the KV write of 65536 tokens 84.3 -> 69.0 us, the
// step's fused draft attention launch 16.9 -> 16.4 us, the fused target launch unchanged
// (its block reads its new keys back after a barrier either way).
template <int G, bool INT8>
__device__ __forceinline__ void store_kv_chunk(uint4 kr, uint4 vr, void* kc, void* vc,
                                               int64_t c_off, uint16_t* ks, uint16_t* vs,
                                               int64_t s_off, int c) {
  typedef uint32_t u32x4_st __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2_st __attribute__((ext_vector_type(2)));
  if constexpr (!INT8) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_st, kr),
                                reinterpret_cast<u32x4_st*>(static_cast<uint16_t*>(kc) + c_off));
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_st, vr),
                                reinterpret_cast<u32x4_st*>(static_cast<uint16_t*>(vc) + c_off));
  } else {
    const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
    const uint32_t vw[4] = {vr.x, vr.y, vr.z, vr.w};
    uint32_t kmax = 0, vmax = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // |bf16| ordering equals integer ordering of the low 15 bits for finite values.
      const uint32_t k0 = kw[i] & 0x7fffu, k1 = (kw[i] >> 16) & 0x7fffu;
      const uint32_t v0 = vw[i] & 0x7fffu, v1 = (vw[i] >> 16) & 0x7fffu;
      kmax = max(kmax, max(k0, k1));
      vmax = max(vmax, max(v0, v1));
    }
    kmax = group_max_u32<G>(kmax);
    vmax = group_max_u32<G>(vmax);
    const float ksc = quant_scale<127>(bf16_to_f32(static_cast<uint16_t>(kmax)));
    const float vsc = quant_scale<127>(bf16_to_f32(static_cast<uint16_t>(vmax)));
    const uint2 kq = quant_pack8_i8(kw, ksc), vq = quant_pack8_i8(vw, vsc);
    __builtin_nontemporal_store(u32x2_st{kq.x, kq.y},
                                reinterpret_cast<u32x2_st*>(static_cast<int8_t*>(kc) + c_off));
    __builtin_nontemporal_store(u32x2_st{vq.x, vq.y},
                                reinterpret_cast<u32x2_st*>(static_cast<int8_t*>(vc) + c_off));
    if (c == 0) {
      ks[s_off] = f32_to_f16(ksc);
      vs[s_off] = f32_to_f16(vsc);
    }
  }
}

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return f32_to_bf16(a) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// neox RoPE (engine/model.py:92-94) on lane c's chunk (elements [8c, 8c + 8)) of a G-lane
// group holding one head vector (D = 8G): element i pairs with i + D/2, which lives in lane
// c ^ (G/2) of the same group, so every lane of the group must run this together.  The
// rotation is rounded to bf16 per element, as the reference's bf16 ops round it.
struct RopeTab {
  uint4 cos, sin;
};
// the table row a position reads: positions outside [0, max_pos) read the nearest row
__device__ __forceinline__ int64_t clamp_pos(int64_t p, int max_pos) {
  return p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p);
}
template <int G>
__device__ __forceinline__ RopeTab rope_tab(const uint16_t* cos, const uint16_t* sin, int64_t stride,
                                            int64_t p, int max_pos, int c) {
  p = clamp_pos(p, max_pos);
  const int i0 = (c < G / 2 ? c : c - G / 2) * 8;
  RopeTab t;
  t.cos = *reinterpret_cast<const uint4*>(cos + p * stride + i0);
  t.sin = *reinterpret_cast<const uint4*>(sin + p * stride + i0);
  return t;
}
template <int G>
__device__ __forceinline__ uint4 rope_chunk(uint4 xr, const RopeTab& t, int c) {
  const bool first = c < G / 2;
  // partner words (elements i +- D/2) from lane c ^ (G/2)
  uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w}, pw[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) pw[e] = __shfl_xor(xw[e], G / 2, COOPT_WAVE);
  const uint32_t cw[4] = {t.cos.x, t.cos.y, t.cos.z, t.cos.w}, sw[4] = {t.sin.x, t.sin.y, t.sin.z, t.sin.w};
  uint32_t yw[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float y[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const float x = bf16_to_f32(static_cast<uint16_t>(xw[e] >> (16 * hh)));
      const float xp = bf16_to_f32(static_cast<uint16_t>(pw[e] >> (16 * hh)));
      const float cs = bf16_to_f32(static_cast<uint16_t>(cw[e] >> (16 * hh)));
      const float sn = bf16_to_f32(static_cast<uint16_t>(sw[e] >> (16 * hh)));
      // first half: x1 c - x2 s; second half: x2 c + x1 s (x = own element, xp = partner)
      y[hh] = first ? fmaf(x, cs, -(xp * sn)) : fmaf(x, cs, xp * sn);
    }
    yw[e] = pack2_bf16(y[0], y[1]);
  }
  return make_uint4(yw[0], yw[1], yw[2], yw[3]);
}

}  // namespace
