// Paged KV write (bf16 copy or fused INT8 quantise) and the symmetric absmax codec.
//
// Quantisation follows kv_tier_manager.quantize (engine/kv_tier_manager.py:21-31) as torch
// executes it on a GPU tensor:
//   amax  = max |x| over the last dim (exact in any format)
//   s32   = max(amax, fp32(1e-8)) * fp32(1/qmax)   -- torch's GPU path turns "tensor / python
//           scalar" into a multiply by the fp32 reciprocal of the scalar
//   code  = int8(clamp(round_half_even(x / s32), -qmax, qmax))   -- IEEE fp32 division
//   scale = fp16(s32), round to nearest even
// Dequantisation (engine/kv_tier_manager.py:34-41): out = dtype(float(code) * float(scale)).
#include "common.h"

namespace {

constexpr float kClampMin = 1e-8f;  // torch converts clamp_min(1e-8) to the tensor's fp32

template <int QMAX>
__device__ __forceinline__ float quant_scale(float amax) {
  return fmaxf(amax, kClampMin) * (1.0f / static_cast<float>(QMAX));
}

template <int QMAX>
__device__ __forceinline__ int quant_code(float x, float s32) {
  float r = rintf(x / s32);
  r = fminf(fmaxf(r, -static_cast<float>(QMAX)), static_cast<float>(QMAX));
  return static_cast<int>(r);
}

// ---------------------------------------------------------------------------------------
// KV write.  One lane per 16-byte chunk (8 bf16) of a (token, head) vector; G = D/8 lanes
// (an aligned power-of-two group inside the wave) cover one vector, and each lane handles
// the same chunk of K and of V, so every load and store is a 16- or 8-byte access.
// ---------------------------------------------------------------------------------------
template <int G, bool INT8>
__global__ __launch_bounds__(256) void kv_write_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t k_ts, int64_t k_hs,
    int64_t v_ts, int64_t v_hs, void* __restrict__ kc, void* __restrict__ vc, int64_t c_bs, int64_t c_ts, int64_t c_hs,
    uint16_t* __restrict__ ks, uint16_t* __restrict__ vs, int64_t s_bs, int64_t s_ts, int64_t s_hs,
    const int64_t* __restrict__ slot_mapping, int T, int Hkv, int block_size, int64_t num_slots) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int c = static_cast<int>(gid % G);
  const int64_t vec = gid / G;
  // Groups are aligned inside the wave, so a whole group leaves together.
  if (vec >= static_cast<int64_t>(T) * Hkv) return;
  const int t = static_cast<int>(vec / Hkv);
  const int h = static_cast<int>(vec % Hkv);
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / block_size;
  const int64_t off = slot % block_size;

  const uint4 kr = *reinterpret_cast<const uint4*>(k + t * k_ts + h * k_hs + c * 8);
  const uint4 vr = *reinterpret_cast<const uint4*>(v + t * v_ts + h * v_hs + c * 8);
  const int64_t c_off = blk * c_bs + off * c_ts + h * c_hs + c * 8;

  if constexpr (!INT8) {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(kc) + c_off) = kr;
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(vc) + c_off) = vr;
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
    uint32_t kq[2] = {0, 0}, vq[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t kb = static_cast<uint16_t>(kw[i / 2] >> (16 * (i & 1)));
      const uint16_t vb = static_cast<uint16_t>(vw[i / 2] >> (16 * (i & 1)));
      const uint32_t kc8 = static_cast<uint32_t>(quant_code<127>(bf16_to_f32(kb), ksc)) & 0xffu;
      const uint32_t vc8 = static_cast<uint32_t>(quant_code<127>(bf16_to_f32(vb), vsc)) & 0xffu;
      kq[i / 4] |= kc8 << (8 * (i & 3));
      vq[i / 4] |= vc8 << (8 * (i & 3));
    }
    *reinterpret_cast<uint2*>(static_cast<int8_t*>(kc) + c_off) = make_uint2(kq[0], kq[1]);
    *reinterpret_cast<uint2*>(static_cast<int8_t*>(vc) + c_off) = make_uint2(vq[0], vq[1]);
    if (c == 0) {
      const int64_t s_off = blk * s_bs + off * s_ts + h * s_hs;
      ks[s_off] = f32_to_f16(ksc);
      vs[s_off] = f32_to_f16(vsc);
    }
  }
}

template <bool INT8>
int launch_kv_write(int G, const uint16_t* k, const uint16_t* v, int64_t k_ts, int64_t k_hs,
                    int64_t v_ts, int64_t v_hs, void* kc, void* vc, int64_t c_bs, int64_t c_ts, int64_t c_hs, uint16_t* ks,
                    uint16_t* vs, int64_t s_bs, int64_t s_ts, int64_t s_hs, const int64_t* slot,
                    int T, int Hkv, int block_size, int64_t num_slots, hipStream_t stream) {
  const int64_t threads = static_cast<int64_t>(T) * Hkv * G;
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
#define COOPT_KVW(GV)                                                                         \
  case GV:                                                                                    \
    hipLaunchKernelGGL((kv_write_kernel<GV, INT8>), grid, dim3(256), 0, stream, k, v, k_ts, k_hs, \
                       v_ts, v_hs, kc, vc, c_bs, c_ts, c_hs, ks, vs, s_bs, s_ts, s_hs, slot, T, Hkv, \
                       block_size, num_slots);                                                \
    break;
  switch (G) {
    COOPT_KVW(1)
    COOPT_KVW(2)
    COOPT_KVW(4)
    COOPT_KVW(8)
    COOPT_KVW(16)
    COOPT_KVW(32)
    COOPT_KVW(64)
    default:
      return COOPT_EINVAL;
  }
#undef COOPT_KVW
  return coopt::check_launch("coopt_kv_write");
}

// ---------------------------------------------------------------------------------------
// Codec over contiguous rows: one wave per row, two elements per lane per step (so an INT4
// byte is produced by one lane).  The row is read twice; the second pass hits the cache.
// ---------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float load_elem(const T* p);
template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }
template <>
__device__ __forceinline__ float load_elem<_Float16>(const _Float16* p) {
  return static_cast<float>(*p);
}
template <>
__device__ __forceinline__ float load_elem<float>(const float* p) { return *p; }

template <typename T, int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(const T* __restrict__ x, int64_t rows,
                                                       int D, uint8_t* __restrict__ q,
                                                       uint16_t* __restrict__ scale) {
  constexpr int QMAX = BITS == 8 ? 127 : 7;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * D;
  float amax = 0.0f;
  for (int i = 2 * lane; i < D; i += 128) {
    amax = fmaxf(amax, fmaxf(fabsf(load_elem(xr + i)), fabsf(load_elem(xr + i + 1))));
  }
  amax = wave_max_f32(amax);
  const float s32 = quant_scale<QMAX>(amax);
  for (int i = 2 * lane; i < D; i += 128) {
    const int c0 = quant_code<QMAX>(load_elem(xr + i), s32);
    const int c1 = quant_code<QMAX>(load_elem(xr + i + 1), s32);
    if constexpr (BITS == 8) {
      const uint16_t pair = static_cast<uint16_t>((c0 & 0xff) | ((c1 & 0xff) << 8));
      *reinterpret_cast<uint16_t*>(q + row * D + i) = pair;
    } else {
      q[row * (D / 2) + i / 2] = static_cast<uint8_t>((c0 + 8) | ((c1 + 8) << 4));
    }
  }
  if (lane == 0) scale[row] = f32_to_f16(s32);
}

template <typename T>
__device__ __forceinline__ void store_elem(T* p, float v);
template <>
__device__ __forceinline__ void store_elem<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16(v); }
template <>
__device__ __forceinline__ void store_elem<_Float16>(_Float16* p, float v) {
  *p = static_cast<_Float16>(v);
}
template <>
__device__ __forceinline__ void store_elem<float>(float* p, float v) { *p = v; }

template <typename T, int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ q,
                                                         const uint16_t* __restrict__ scale,
                                                         int64_t rows, int D, T* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float s = f16_to_f32(scale[row]);
  for (int i = 2 * lane; i < D; i += 128) {
    int c0, c1;
    if constexpr (BITS == 8) {
      const uint16_t pair = *reinterpret_cast<const uint16_t*>(q + row * D + i);
      c0 = static_cast<int8_t>(pair & 0xff);
      c1 = static_cast<int8_t>(pair >> 8);
    } else {
      const uint8_t b = q[row * (D / 2) + i / 2];
      c0 = static_cast<int>(b & 0x0f) - 8;
      c1 = static_cast<int>(b >> 4) - 8;
    }
    store_elem(out + row * D + i, static_cast<float>(c0) * s);
    store_elem(out + row * D + i + 1, static_cast<float>(c1) * s);
  }
}

}  // namespace

extern "C" int coopt_kv_write(int cache_dtype, const void* k, const void* v, int64_t k_tok_stride,
                              int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                              void* k_cache, void* v_cache,
                              int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                              void* k_scale, void* v_scale, int64_t s_blk_stride,
                              int64_t s_tok_stride, int64_t s_head_stride,
                              const int64_t* slot_mapping, int T, int Hkv, int D, int block_size,
                              int64_t num_blocks, coopt_stream_t stream) {
  COOPT_REQUIRE(cache_dtype == COOPT_DT_BF16 || cache_dtype == COOPT_DT_I8,
                "cache_dtype must be COOPT_DT_BF16 or COOPT_DT_I8");
  COOPT_REQUIRE(T >= 0 && Hkv > 0 && block_size > 0 && num_blocks > 0, "bad sizes");
  COOPT_REQUIRE(D % 8 == 0 && D >= 8 && D <= 512 && ((D / 8) & (D / 8 - 1)) == 0,
                "D must be 8 * a power of two, at most 512");
  if (T == 0) return COOPT_OK;
  COOPT_REQUIRE(k && v && k_cache && v_cache && slot_mapping, "null pointer");
  COOPT_REQUIRE(coopt::aligned16(k) && coopt::aligned16(v) && k_tok_stride % 8 == 0 &&
                    k_head_stride % 8 == 0 && v_tok_stride % 8 == 0 && v_head_stride % 8 == 0,
                "k/v rows must be 16-byte aligned (strides multiples of 8 elements)");
  const bool int8 = cache_dtype == COOPT_DT_I8;
  if (int8) {
    COOPT_REQUIRE(k_scale && v_scale, "INT8 cache needs k_scale and v_scale");
    COOPT_REQUIRE((reinterpret_cast<uintptr_t>(k_cache) & 7u) == 0 &&
                      (reinterpret_cast<uintptr_t>(v_cache) & 7u) == 0 && c_blk_stride % 8 == 0 &&
                      c_tok_stride % 8 == 0 && c_head_stride % 8 == 0,
                  "INT8 cache rows must be 8-byte aligned");
    COOPT_REQUIRE((reinterpret_cast<uintptr_t>(k_scale) & 1u) == 0 &&
                      (reinterpret_cast<uintptr_t>(v_scale) & 1u) == 0,
                  "scales must be 2-byte aligned");
  } else {
    COOPT_REQUIRE(coopt::aligned16(k_cache) && coopt::aligned16(v_cache) &&
                      c_blk_stride % 8 == 0 && c_tok_stride % 8 == 0 && c_head_stride % 8 == 0,
                  "bf16 cache rows must be 16-byte aligned");
  }
  coopt::clear_error();
  const int64_t num_slots = num_blocks * block_size;
  auto s = static_cast<hipStream_t>(stream);
  const auto* kp = static_cast<const uint16_t*>(k);
  const auto* vp = static_cast<const uint16_t*>(v);
  if (int8)
    return launch_kv_write<true>(D / 8, kp, vp, k_tok_stride, k_head_stride, v_tok_stride,
                                 v_head_stride, k_cache, v_cache,
                                 c_blk_stride, c_tok_stride, c_head_stride,
                                 static_cast<uint16_t*>(k_scale), static_cast<uint16_t*>(v_scale),
                                 s_blk_stride, s_tok_stride, s_head_stride, slot_mapping, T, Hkv,
                                 block_size, num_slots, s);
  return launch_kv_write<false>(D / 8, kp, vp, k_tok_stride, k_head_stride, v_tok_stride,
                                v_head_stride, k_cache, v_cache,
                                c_blk_stride, c_tok_stride, c_head_stride, nullptr, nullptr, 0, 0,
                                0, slot_mapping, T, Hkv, block_size, num_slots, s);
}

extern "C" int coopt_quantize(int bits, int in_dtype, const void* x, int64_t rows, int D, void* q,
                              void* scale, coopt_stream_t stream) {
  COOPT_REQUIRE(bits == 8 || bits == 4, "bits must be 8 or 4");
  COOPT_REQUIRE(rows >= 0 && D > 0 && D % 2 == 0 && D <= 4096, "D must be even, <= 4096");
  if (rows == 0) return COOPT_OK;
  COOPT_REQUIRE(x && q && scale, "null pointer");
  COOPT_REQUIRE((reinterpret_cast<uintptr_t>(q) & 1u) == 0 || bits == 4, "q must be 2-byte aligned");
  coopt::clear_error();
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  auto s = static_cast<hipStream_t>(stream);
  auto* qp = static_cast<uint8_t*>(q);
  auto* sp = static_cast<uint16_t*>(scale);
#define COOPT_Q(T, B) \
  hipLaunchKernelGGL((quantize_kernel<T, B>), grid, dim3(256), 0, s, static_cast<const T*>(x), rows, D, qp, sp)
  switch (in_dtype) {
    case COOPT_DT_BF16:
      if (bits == 8) COOPT_Q(uint16_t, 8); else COOPT_Q(uint16_t, 4);
      break;
    case COOPT_DT_F16:
      if (bits == 8) COOPT_Q(_Float16, 8); else COOPT_Q(_Float16, 4);
      break;
    case COOPT_DT_F32:
      if (bits == 8) COOPT_Q(float, 8); else COOPT_Q(float, 4);
      break;
    default:
      coopt::set_error("coopt_quantize: in_dtype must be BF16, F16 or F32");
      return COOPT_EINVAL;
  }
#undef COOPT_Q
  return coopt::check_launch("coopt_quantize");
}

extern "C" int coopt_dequantize(int bits, const void* q, const void* scale, int64_t rows, int D,
                                int out_dtype, void* out, coopt_stream_t stream) {
  COOPT_REQUIRE(bits == 8 || bits == 4, "bits must be 8 or 4");
  COOPT_REQUIRE(rows >= 0 && D > 0 && D % 2 == 0 && D <= 4096, "D must be even, <= 4096");
  if (rows == 0) return COOPT_OK;
  COOPT_REQUIRE(q && scale && out, "null pointer");
  coopt::clear_error();
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  auto s = static_cast<hipStream_t>(stream);
  const auto* qp = static_cast<const uint8_t*>(q);
  const auto* sp = static_cast<const uint16_t*>(scale);
#define COOPT_DQ(T, B) \
  hipLaunchKernelGGL((dequantize_kernel<T, B>), grid, dim3(256), 0, s, qp, sp, rows, D, static_cast<T*>(out))
  switch (out_dtype) {
    case COOPT_DT_BF16:
      if (bits == 8) COOPT_DQ(uint16_t, 8); else COOPT_DQ(uint16_t, 4);
      break;
    case COOPT_DT_F16:
      if (bits == 8) COOPT_DQ(_Float16, 8); else COOPT_DQ(_Float16, 4);
      break;
    case COOPT_DT_F32:
      if (bits == 8) COOPT_DQ(float, 8); else COOPT_DQ(float, 4);
      break;
    default:
      coopt::set_error("coopt_dequantize: out_dtype must be BF16, F16 or F32");
      return COOPT_EINVAL;
  }
#undef COOPT_DQ
  return coopt::check_launch("coopt_dequantize");
}
