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
#include "kv_store.h"

namespace {

template <int G, bool INT8>
__global__ __launch_bounds__(256) void kv_write_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t k_ts, int64_t k_hs,
    int64_t v_ts, int64_t v_hs, void* __restrict__ kc, void* __restrict__ vc, int64_t c_bs, int64_t c_ts, int64_t c_hs,
    uint16_t* __restrict__ ks, uint16_t* __restrict__ vs, int64_t s_bs, int64_t s_ts, int64_t s_hs,
    const int64_t* __restrict__ slot_mapping, int T, int bs_shift, int block_size, int64_t num_slots) {
  // grid: x covers T tokens x G lanes (32-bit, checked by the host), y the KV head
  const int lid = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  const int c = lid & (G - 1);
  const int t = lid / G;
  // Groups are aligned inside the wave, so a whole group leaves together.
  if (t >= T) return;
  const int h = blockIdx.y;
  // The K and V chunks load with the slot (none depends on another); the empty asm takes all
  // three, so the compiler neither sinks the K / V loads past the slot test nor waits for the
  // slot before issuing them: one memory round trip instead of two.
  const uint4 kr = *reinterpret_cast<const uint4*>(k + t * k_ts + h * k_hs + c * 8);
  const uint4 vr = *reinterpret_cast<const uint4*>(v + t * v_ts + h * v_hs + c * 8);
  const int64_t slot = slot_mapping[t];
  asm volatile("" ::"v"(kr.x), "v"(kr.y), "v"(kr.z), "v"(kr.w), "v"(vr.x), "v"(vr.y), "v"(vr.z),
               "v"(vr.w), "v"(slot));
  if (slot < 0 || slot >= num_slots) return;
  // power-of-two block sizes (bs_shift >= 0) take a shift and a mask
  const int64_t blk = bs_shift >= 0 ? slot >> bs_shift : slot / block_size;
  const int64_t off = bs_shift >= 0 ? slot & ((int64_t{1} << bs_shift) - 1) : slot % block_size;

  const int64_t c_off = blk * c_bs + off * c_ts + h * c_hs + c * 8;
  store_kv_chunk<G, INT8>(kr, vr, kc, vc, c_off, ks, vs, blk * s_bs + off * s_ts + h * s_hs, c);
}

// ---------------------------------------------------------------------------------------
// qkv epilogue: the chain  F.linear(h, qkv).split -> rotary_embedding(q, k) ->
// reshape_and_cache_flash(k, v)  of engine/model.py:238-243 after the qkv projection, in one
// launch.  A G-lane group (G = D/8) owns one (token, head) vector of the T x (Hq + Hkv) q and
// k heads; k groups also carry their token's v head.  The input row is either the bf16 qkv
// output or the fp32 split-K partials of the projection (reduced here in the order
// coopt_linear's reduction uses, then rounded to bf16 as it would be).  RoPE (neox halves)
// pairs element i with i + D/2, which lives in lane c ^ (G/2) of the same group: one
// shuffle per word.  q heads go to q_out; k (rotated) and v go to the paged cache exactly as
// coopt_kv_write stores them, and rows with slot < 0 write no cache entry.
// ---------------------------------------------------------------------------------------
struct QkvArgs {
  const uint16_t* qkv;
  int64_t qkv_ts;
  const float* part;
  int ks;
  int64_t slice;
  const int64_t* pos;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t tab_stride;
  int max_pos;
  uint16_t* q_out;
  int64_t q_ts, q_hs;
  void* kc;
  void* vc;
  int64_t c_bs, c_ts, c_hs;
  uint16_t* k_scale;
  uint16_t* v_scale;
  int64_t s_bs, s_ts, s_hs;
  const int64_t* slot_mapping;
  int T, Hq, Hkv, D, block_size;
  int64_t num_slots;
  int bs_shift;  // log2(block_size) when it is a power of two, else -1
};


// Elements [col, col + 8) of row t: bf16 from the qkv output, or bf16(sum of the partials).
__device__ __forceinline__ uint4 qkv_chunk(const QkvArgs& a, int t, int64_t col) {
  if (a.part) {
    const float* p = a.part + static_cast<int64_t>(t) * (a.Hq + 2 * a.Hkv) * a.D + col;
    const float4 lo = sum_partials4(p, a.ks, a.slice), hi = sum_partials4(p + 4, a.ks, a.slice);
    return make_uint4(pack2_bf16(lo.x, lo.y), pack2_bf16(lo.z, lo.w), pack2_bf16(hi.x, hi.y),
                      pack2_bf16(hi.z, hi.w));
  }
  return *reinterpret_cast<const uint4*>(a.qkv + static_cast<int64_t>(t) * a.qkv_ts + col);
}

// Elements [col, col + 8) of row t, loaded now and returned by get(): with KS > 0 the fp32
// partials (slice count bounded by KS at compile time, every load unconditional), else
// qkv_chunk's bf16 row or runtime-bounded partials.
template <int KS>
struct QkvChunk {
  Partials4<(KS > 0 ? KS : 1)> lo, hi;
  uint4 raw;
  __device__ __forceinline__ void load(const QkvArgs& a, int t, int64_t col) {
    if constexpr (KS > 0) {
      const float* p = a.part + static_cast<int64_t>(t) * (a.Hq + 2 * a.Hkv) * a.D + col;
      lo.load(p, a.ks, a.slice);
      hi.load(p + 4, a.ks, a.slice);
    } else {
      raw = qkv_chunk(a, t, col);
    }
  }
  __device__ __forceinline__ uint4 get(const QkvArgs& a) const {
    if constexpr (KS > 0) {
      const float4 l = lo.sum(a.ks), h = hi.sum(a.ks);
      return make_uint4(pack2_bf16(l.x, l.y), pack2_bf16(l.z, l.w), pack2_bf16(h.x, h.y),
                        pack2_bf16(h.z, h.w));
    } else {
      return raw;
    }
  }
};

template <int G, bool INT8, int KS>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(QkvArgs a) {
  // grid: x covers T tokens x G lanes (32-bit, checked by the host), y the q / k head
  const int lid = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  const int c = lid & (G - 1);
  const int t = lid / G;
  if (t >= a.T) return;  // whole groups leave together
  const int h = blockIdx.y;
  const bool is_k = h >= a.Hq;  // uniform over the block
  const int hk = h - a.Hq;
  const int D = G * 8;
  // Issue order: the position (and slot), then the row's chunks; the wait for the position
  // (the cos/sin addresses) then leaves the chunk loads in flight.
  int64_t p = a.pos[t];
  const int64_t slot = is_k ? a.slot_mapping[t] : -1;
  QkvChunk<KS> xc, vc;
  xc.load(a, t, static_cast<int64_t>(h) * D + c * 8);
  if (is_k) vc.load(a, t, static_cast<int64_t>(a.Hq + a.Hkv + hk) * D + c * 8);
  const RopeTab rt = rope_tab<G>(a.cos, a.sin, a.tab_stride, p, a.max_pos, c);
  const uint4 yr = rope_chunk<G>(xc.get(a), rt, c);
  if (!is_k) {
    *reinterpret_cast<uint4*>(a.q_out + t * a.q_ts + h * a.q_hs + c * 8) = yr;
    return;
  }
  if (slot < 0 || slot >= a.num_slots) return;  // padding row: the group leaves together
  const uint4 vr = vc.get(a);
  const int64_t blk = a.bs_shift >= 0 ? slot >> a.bs_shift : slot / a.block_size;
  const int64_t off = a.bs_shift >= 0 ? slot & ((int64_t{1} << a.bs_shift) - 1) : slot % a.block_size;
  store_kv_chunk<G, INT8>(yr, vr, a.kc, a.vc, blk * a.c_bs + off * a.c_ts + hk * a.c_hs + c * 8,
                          a.k_scale, a.v_scale, blk * a.s_bs + off * a.s_ts + hk * a.s_hs, c);
}

template <bool INT8>
int launch_kv_write(int G, const uint16_t* k, const uint16_t* v, int64_t k_ts, int64_t k_hs,
                    int64_t v_ts, int64_t v_hs, void* kc, void* vc, int64_t c_bs, int64_t c_ts, int64_t c_hs, uint16_t* ks,
                    uint16_t* vs, int64_t s_bs, int64_t s_ts, int64_t s_hs, const int64_t* slot,
                    int T, int Hkv, int block_size, int64_t num_slots, hipStream_t stream) {
  const int64_t lanes = static_cast<int64_t>(T) * G;
  COOPT_REQUIRE(lanes <= 0x7fffff00LL && Hkv <= 65535, "T * D / 8 must stay below 2^31, Hkv <= 65535");
  const dim3 grid(static_cast<unsigned>((lanes + 255) / 256), static_cast<unsigned>(Hkv));
  const int bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
#define COOPT_KVW(GV)                                                                         \
  case GV:                                                                                    \
    hipLaunchKernelGGL((kv_write_kernel<GV, INT8>), grid, dim3(256), 0, stream, k, v, k_ts, k_hs, \
                       v_ts, v_hs, kc, vc, c_bs, c_ts, c_hs, ks, vs, s_bs, s_ts, s_hs, slot, T, \
                       bs_shift, block_size, num_slots);                                      \
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
  const float r32 = __builtin_amdgcn_rcpf(s32);
  for (int i = 2 * lane; i < D; i += 128) {
    const int c0 = quant_code<QMAX>(load_elem(xr + i), s32, r32);
    const int c1 = quant_code<QMAX>(load_elem(xr + i + 1), s32, r32);
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

// ---------------------------------------------------------------------------------------
// Swap codec (engine/kv_tier_manager.py:93-101 and :113-119).  swap_out gathers whole cache
// blocks by id and quantises them into a contiguous [n_ids, block_size, Hkv, D(/2)] buffer --
// quantize(cache[blocks], bits) in one launch; swap_in dequantises such a buffer and scatters
// it into blocks -- cache[blocks] = dequantize(q, s, bits, cache.dtype).  G = D/8 lanes per
// (token, head) vector, 8 elements each.  An INT8 cache already holds codes and scales: its
// blocks are copied as they are (bits 8 only).  Ids outside [0, num_blocks) read as zeros
// (swap_out) or are skipped (swap_in).
// ---------------------------------------------------------------------------------------
template <int BITS>
struct SwapElt {  // bytes of 8 elements in the swapped format
  static constexpr int kBytes = BITS == 16 ? 16 : (BITS == 8 ? 8 : 4);
};

// Up to kMaxSwapCaches caches (e.g. the K and V caches of every layer) of one shape and
// strides, swapped by one launch: grid.y picks the cache, and cache i's swapped rows sit at
// q + i * q_stride bytes and scale + i * s_stride elements.
constexpr int kMaxSwapCaches = 64;
struct CacheSet {
  const void* c[kMaxSwapCaches];
  uint16_t* s[kMaxSwapCaches];  // INT8 caches: their fp16 scale caches
};

// One workgroup moves one slab of U * kSwapThreads chunks (of 8 elements) of one swapped
// block for one cache: a thread takes U chunks, kSwapThreads apart, and issues every load
// before it uses the first, so it keeps U loads in flight rather than one (one 16-byte load
// per thread left the stream at about half the HBM rate).  U = 4 for swap_out and 2 for
// swap_in measured best (32 layers' K and V of a 4096-token sequence: 250 -> 190 us and
// 224 -> 145 us; 8 was slower at both, and 4 left one layer's swap_out 0.4 us slower than
// one chunk per thread, which launches too small to fill the GPU therefore keep).
// Nothing in a slab branches: a load under a branch is waited for where the branch joins,
// and the compiler sinks a load into the branch of its only store.  So a chunk index past
// the block stands for the same chunk of the block's first vector (its G-lane group stays
// whole) and that lane stores the same bytes as the lane that owns the chunk; a vector's
// scale is stored by its chunk-0 lane (a store under a branch holds nothing up).
// Chunk idx of a block is (token t, head h, chunk c) with idx = (t * Hkv + h) * G + c, the
// order of the swapped rows, so the swapped side is read or written contiguously.
constexpr int kSwapThreads = 256;
constexpr int kSwapOutU = 4;
constexpr int kSwapInU = 2;
// Two-chunks-a-lane forms (INT8 out of bf16): pairs per thread of swap_out and of the codec.
constexpr int kSwapPairOutU = 4;
constexpr int kCodecPairU = 2;
constexpr int64_t kSwapSmallGrid = 2048;

template <int N>
struct SwapVec;  // the register type of N bytes
template <>
struct SwapVec<16> { using T = uint4; };
template <>
struct SwapVec<8> { using T = uint2; };
template <>
struct SwapVec<4> { using T = uint32_t; };

// The chunk of round u of this thread in the slab that starts at chunk `base` of its block.
template <int G>
__device__ __forceinline__ int swap_chunk(int base, int u, int nchunk) {
  const int idx = base + u * kSwapThreads + static_cast<int>(threadIdx.x);
  return idx < nchunk ? idx : idx % G;
}

// The swapped form of one 8-element bf16 chunk (words w, element 2i in the low half of w[i])
// of a G-lane group's vector: kv_tier_manager.quantize per vector (engine/kv_tier_manager.py:
// 21-31) -- INT8 codes in lo / hi, or INT4 nibbles (even element low, +8 offset) in lo --
// and the vector's fp16 scale.  Every lane of the group must call it together.
struct QuantChunk {
  uint32_t lo, hi;
  uint16_t scale;
};
template <int G, int BITS>
__device__ __forceinline__ QuantChunk quant_chunk(const uint32_t (&w)[4]) {
  constexpr int QMAX = BITS == 8 ? 127 : 7;
  uint32_t amax = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) amax = max(amax, max(w[e] & 0x7fffu, (w[e] >> 16) & 0x7fffu));
  amax = group_max_u32<G>(amax);
  const float s32 = quant_scale<QMAX>(bf16_to_f32(static_cast<uint16_t>(amax)));
  QuantChunk r{0, 0, f32_to_f16(s32)};
  if constexpr (BITS == 8) {
    const uint2 p = quant_pack8_i8(w, s32);
    r.lo = p.x;
    r.hi = p.y;
  } else {
    int code[8];
    quant_codes8<QMAX>(w, s32, code);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r.lo |= ((static_cast<uint32_t>(code[2 * j] + 8) | (static_cast<uint32_t>(code[2 * j + 1] + 8) << 4)) & 0xffu) << (8 * j);
  }
  return r;
}

// bf16(float(code) * float(scale)) of one chunk's 8 codes (INT8 in lo / hi, or INT4 nibbles
// in lo): dequantize, engine/kv_tier_manager.py:34-41.  The product is exact.
template <int BITS>
__device__ __forceinline__ uint4 dequant_chunk(uint32_t lo, uint32_t hi, uint16_t scale16) {
  const float sc = f16_to_f32(scale16);
  int code[8];
  if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) code[e] = static_cast<int8_t>(((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xffu);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t byte = (lo >> (8 * j)) & 0xffu;
      code[2 * j] = static_cast<int>(byte & 0x0fu) - 8;
      code[2 * j + 1] = static_cast<int>(byte >> 4) - 8;
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = f32_to_bf16(static_cast<float>(code[2 * e]) * sc) |
           (static_cast<uint32_t>(f32_to_bf16(static_cast<float>(code[2 * e + 1]) * sc)) << 16);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 16 bytes of a bf16 cache read by swap_out, with the nontemporal hint: the blocks are read
// once.  Alternated with plain loads on MI355X, 32 layers' swap_out went 164-167 -> 160-162 us;
// the row quantiser, which reads its input the same way, went 22.0 -> 23.1 us with the hint
// and keeps plain loads.
__device__ __forceinline__ uint4 ld16_stream(const uint16_t* p) {
  typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_v*>(p)));
}

// 16 bytes of bf16 written by swap_in or the row dequantiser, with the nontemporal hint: the
// output is not read again by the same launch.  Alternated with plain stores on MI355X, 32
// layers' swap_in went 147-150 -> 136-141 us and 64 MiB of dequantised rows 15.8 -> 15.2 us.
__device__ __forceinline__ void st16_stream(void* p, uint4 v) {
  typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_v, v), reinterpret_cast<u32x4_v*>(p));
}

// 8 bytes of codes written by the row quantiser, with the nontemporal hint (its 16-byte form
// uses st16_stream).  Alternated with plain stores on MI355X, 64 MiB of bf16 rows went
// 22.0-22.3 -> 20.5 us; swap_out's code stores measured the same either way and stay plain.
__device__ __forceinline__ void st8_stream(void* p, uint32_t lo, uint32_t hi) {
  typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(u32x2_v{lo, hi}, reinterpret_cast<u32x2_v*>(p));
}

template <int G, int BITS, bool SRC8, int U = kSwapOutU>
__global__ __launch_bounds__(kSwapThreads) void swap_out_kernel(
    CacheSet cs, int64_t c_bs, int64_t c_ts, int64_t c_hs, int64_t s_bs, int64_t s_ts, int64_t s_hs,
    const int64_t* __restrict__ ids, int slabs, int bs, int Hkv, int64_t num_blocks,
    unsigned char* __restrict__ q, uint16_t* __restrict__ scale, int64_t q_stride,
    int64_t s_stride) {
  const void* __restrict__ cache = cs.c[blockIdx.y];
  const uint16_t* __restrict__ cscale = cs.s[blockIdx.y];
  constexpr int kOut = SwapElt<BITS>::kBytes;
  using In = typename SwapVec<SRC8 ? 8 : 16>::T;
  const int i = static_cast<int>(blockIdx.x) / slabs;
  const int base = (static_cast<int>(blockIdx.x) - i * slabs) * (U * kSwapThreads);
  const int per_blk = bs * Hkv;
  const int nchunk = per_blk * G;
  const int64_t vec0 = static_cast<int64_t>(i) * per_blk;
  q += blockIdx.y * q_stride + vec0 * G * kOut;
  scale += blockIdx.y * s_stride + vec0;
  const int64_t blk = ids[i];
  if (blk < 0 || blk >= num_blocks) {  // uniform: the block's rows read as zeros
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = swap_chunk<G>(base, u, nchunk);
      unsigned char* qo = q + static_cast<int64_t>(idx) * kOut;
      if constexpr (kOut == 16) *reinterpret_cast<uint4*>(qo) = make_uint4(0, 0, 0, 0);
      else if constexpr (kOut == 8) *reinterpret_cast<uint2*>(qo) = make_uint2(0, 0);
      else *reinterpret_cast<uint32_t*>(qo) = 0;
      if (BITS != 16 && idx % G == 0) scale[idx / G] = 0;
    }
    return;
  }
  In x[U];
  uint16_t xs[U];  // an INT8 cache: the vector's scale
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    const int v = idx / G, c = idx % G;
    const int t = v / Hkv, h = v - t * Hkv;
    const int64_t off = blk * c_bs + t * c_ts + h * c_hs + c * 8;
    if constexpr (SRC8) {
      x[u] = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(cache) + off);
      xs[u] = cscale[blk * s_bs + t * s_ts + h * s_hs];
    } else {
      x[u] = ld16_stream(static_cast<const uint16_t*>(cache) + off);
    }
  }
  // keeps the scheduler from moving each load down to its store (the copying forms have no
  // other work between them)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    unsigned char* qo = q + static_cast<int64_t>(idx) * kOut;
    if constexpr (SRC8) {
      *reinterpret_cast<uint2*>(qo) = make_uint2(x[u].x, x[u].y);
      if (idx % G == 0) scale[idx / G] = xs[u];
    } else if constexpr (BITS == 16) {
      *reinterpret_cast<uint4*>(qo) = make_uint4(x[u].x, x[u].y, x[u].z, x[u].w);
    } else {
      const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
      const QuantChunk r = quant_chunk<G, BITS>(w);
      if constexpr (BITS == 8) *reinterpret_cast<uint2*>(qo) = make_uint2(r.lo, r.hi);
      else *reinterpret_cast<uint32_t*>(qo) = r.lo;
      if (idx % G == 0) scale[idx / G] = r.scale;
    }
  }
}

// swap_out of bf16 caches at 8 bits with two chunks a lane (G2 = G / 2 lanes a vector): a lane
// loads 32 contiguous bytes of its vector and stores its 16 codes as one 16-byte word.  Same
// slab scheme, wrap rule and output as swap_out_kernel<2 G2, 8, false>.  32 layers' K and V of
// a 4096-token sequence: 179 -> 163 us against one chunk a lane.
template <int G2, int U = kSwapPairOutU>
__global__ __launch_bounds__(kSwapThreads) void swap_out_pair_kernel(
    CacheSet cs, int64_t c_bs, int64_t c_ts, int64_t c_hs, const int64_t* __restrict__ ids,
    int slabs, int bs, int Hkv, int64_t num_blocks, unsigned char* __restrict__ q,
    uint16_t* __restrict__ scale, int64_t q_stride, int64_t s_stride) {
  const uint16_t* __restrict__ cache = static_cast<const uint16_t*>(cs.c[blockIdx.y]);
  const int i = static_cast<int>(blockIdx.x) / slabs;
  const int base = (static_cast<int>(blockIdx.x) - i * slabs) * (U * kSwapThreads);
  const int per_blk = bs * Hkv;
  const int npair = per_blk * G2;
  const int64_t vec0 = static_cast<int64_t>(i) * per_blk;
  q += blockIdx.y * q_stride + vec0 * G2 * 16;
  scale += blockIdx.y * s_stride + vec0;
  const int64_t blk = ids[i];
  if (blk < 0 || blk >= num_blocks) {  // uniform: the block's rows read as zeros
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = swap_chunk<G2>(base, u, npair);
      *reinterpret_cast<uint4*>(q + static_cast<int64_t>(idx) * 16) = make_uint4(0, 0, 0, 0);
      if (idx % G2 == 0) scale[idx / G2] = 0;
    }
    return;
  }
  uint4 xa[U], xb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G2>(base, u, npair);
    const int v = idx / G2, c = idx % G2;
    const int t = v / Hkv, h = v - t * Hkv;
    const uint16_t* src = cache + blk * c_bs + t * c_ts + h * c_hs + c * 16;
    xa[u] = ld16_stream(src);
    xb[u] = ld16_stream(src + 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // as in swap_out_kernel
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G2>(base, u, npair);
    const QuantPair r = quant_pair8<G2>(xa[u], xb[u]);
    *reinterpret_cast<uint4*>(q + static_cast<int64_t>(idx) * 16) = r.codes;
    if (idx % G2 == 0) scale[idx / G2] = r.scale;
  }
}

template <int G, int BITS, bool DST8, int U = kSwapInU>
__global__ __launch_bounds__(kSwapThreads) void swap_in_kernel(
    const unsigned char* __restrict__ q, const uint16_t* __restrict__ scale, int64_t q_stride,
    int64_t s_stride, const int64_t* __restrict__ ids, int slabs, int bs, int Hkv,
    int64_t num_blocks, CacheSet cs, int64_t c_bs, int64_t c_ts, int64_t c_hs, int64_t s_bs,
    int64_t s_ts, int64_t s_hs) {
  void* __restrict__ cache = const_cast<void*>(cs.c[blockIdx.y]);
  uint16_t* __restrict__ cscale = cs.s[blockIdx.y];
  constexpr int kIn = SwapElt<BITS>::kBytes;
  using In = typename SwapVec<kIn>::T;
  const int i = static_cast<int>(blockIdx.x) / slabs;
  const int base = (static_cast<int>(blockIdx.x) - i * slabs) * (U * kSwapThreads);
  const int per_blk = bs * Hkv;
  const int nchunk = per_blk * G;
  const int64_t blk = ids[i];
  if (blk < 0 || blk >= num_blocks) return;  // uniform: skipped
  const int64_t vec0 = static_cast<int64_t>(i) * per_blk;
  q += blockIdx.y * q_stride + vec0 * G * kIn;
  scale += blockIdx.y * s_stride + vec0;
  In r[U];
  uint16_t sv[U];  // the vector's scale
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    r[u] = *reinterpret_cast<const In*>(q + static_cast<int64_t>(idx) * kIn);
    sv[u] = BITS != 16 ? scale[idx / G] : 0;
  }
  __builtin_amdgcn_sched_barrier(0);  // as in swap_out_kernel
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    const int v = idx / G, c = idx % G;
    const int t = v / Hkv, h = v - t * Hkv;
    const int64_t off = blk * c_bs + t * c_ts + h * c_hs + c * 8;
    if constexpr (DST8) {
      *reinterpret_cast<uint2*>(static_cast<int8_t*>(cache) + off) = make_uint2(r[u].x, r[u].y);
      cscale[blk * s_bs + t * s_ts + h * s_hs] = sv[u];
    } else if constexpr (BITS == 16) {
      *reinterpret_cast<uint4*>(static_cast<uint16_t*>(cache) + off) =
          make_uint4(r[u].x, r[u].y, r[u].z, r[u].w);
    } else {
      uint4 o;
      if constexpr (BITS == 8) o = dequant_chunk<8>(r[u].x, r[u].y, sv[u]);
      else o = dequant_chunk<4>(r[u], 0, sv[u]);
      st16_stream(static_cast<uint16_t*>(cache) + off, o);
    }
  }
}

// The codec over contiguous bf16 rows of D = 8G elements, its common case: the swap kernels'
// slab scheme over chunk idx = row * G + c (the rows form one block of nchunk chunks).
template <int G, int BITS, int U = kSwapOutU>
__global__ __launch_bounds__(kSwapThreads) void quantize_rows_kernel(
    const uint16_t* __restrict__ x, int nchunk, unsigned char* __restrict__ q,
    uint16_t* __restrict__ scale) {
  constexpr int kOut = SwapElt<BITS>::kBytes;
  const int base = static_cast<int>(blockIdx.x) * (U * kSwapThreads);
  uint4 xv[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    xv[u] = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(swap_chunk<G>(base, u, nchunk)) * 8);
  __builtin_amdgcn_sched_barrier(0);  // as in swap_out_kernel
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    const uint32_t w[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
    const QuantChunk r = quant_chunk<G, BITS>(w);
    unsigned char* qo = q + static_cast<int64_t>(idx) * kOut;
    if constexpr (BITS == 8) st8_stream(qo, r.lo, r.hi);
    else *reinterpret_cast<uint32_t*>(qo) = r.lo;
    if (idx % G == 0) scale[idx / G] = r.scale;
  }
}

// quantize_rows_kernel at 8 bits with two chunks a lane (G2 = D / 16 lanes a row, 16-byte
// code stores), over pair idx = row * G2 + c.  64 MiB of bf16 rows: 23.4 -> 22.1 us.
template <int G2, int U = kCodecPairU>
__global__ __launch_bounds__(kSwapThreads) void quantize_rows_pair_kernel(
    const uint16_t* __restrict__ x, int npair, unsigned char* __restrict__ q,
    uint16_t* __restrict__ scale) {
  const int base = static_cast<int>(blockIdx.x) * (U * kSwapThreads);
  uint4 xa[U], xb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint16_t* src = x + static_cast<int64_t>(swap_chunk<G2>(base, u, npair)) * 16;
    xa[u] = *reinterpret_cast<const uint4*>(src);
    xb[u] = *reinterpret_cast<const uint4*>(src + 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // as in swap_out_kernel
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G2>(base, u, npair);
    const QuantPair r = quant_pair8<G2>(xa[u], xb[u]);
    st16_stream(q + static_cast<int64_t>(idx) * 16, r.codes);
    if (idx % G2 == 0) scale[idx / G2] = r.scale;
  }
}

template <int G, int BITS, int U = kSwapInU>
__global__ __launch_bounds__(kSwapThreads) void dequantize_rows_kernel(
    const unsigned char* __restrict__ q, const uint16_t* __restrict__ scale, int nchunk,
    uint16_t* __restrict__ out) {
  constexpr int kIn = SwapElt<BITS>::kBytes;
  using In = typename SwapVec<kIn>::T;
  const int base = static_cast<int>(blockIdx.x) * (U * kSwapThreads);
  In r[U];
  uint16_t sv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    r[u] = *reinterpret_cast<const In*>(q + static_cast<int64_t>(idx) * kIn);
    sv[u] = scale[idx / G];
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int idx = swap_chunk<G>(base, u, nchunk);
    uint4 o;
    if constexpr (BITS == 8) o = dequant_chunk<8>(r[u].x, r[u].y, sv[u]);
    else o = dequant_chunk<4>(r[u], 0, sv[u]);
    st16_stream(out + static_cast<int64_t>(idx) * 8, o);
  }
}

// Launches the row codec when the call fits it (bf16 rows, D = 8G with G a power of two up to
// 64, aligned buffers, enough chunks to fill the GPU); returns false to leave the call to the
// general kernels.
bool launch_rows_codec(bool quant, int bits, const void* x, int64_t rows, int D, void* q,
                       const void* scale, hipStream_t s) {
  const int G = D / 8;
  if (D % 8 != 0 || G > 64 || (G & (G - 1)) != 0) return false;
  const int U = quant ? kSwapOutU : kSwapInU;
  const int64_t nchunk = rows * G;
  if (nchunk > INT32_MAX - U * kSwapThreads) return false;
  const int64_t grid = (nchunk + U * kSwapThreads - 1) / (U * kSwapThreads);
  if (grid < kSwapSmallGrid) return false;
  const int qal = bits == 8 ? 8 : 4;
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(q) % qal) != 0 ||
      (reinterpret_cast<uintptr_t>(scale) & 1u) != 0)
    return false;
  const int n = static_cast<int>(nchunk);
  if (quant && bits == 8 && G >= 2 && (reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
    // two chunks a lane (16-byte code stores); 16-byte aligned codes
    const int np = n / 2;
    const dim3 g2(static_cast<unsigned>((np + kCodecPairU * kSwapThreads - 1) / (kCodecPairU * kSwapThreads)));
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    unsigned char* qp = static_cast<unsigned char*>(q);
    uint16_t* sp = static_cast<uint16_t*>(const_cast<void*>(scale));
    switch (G / 2) {
      case 1: hipLaunchKernelGGL((quantize_rows_pair_kernel<1>), g2, dim3(kSwapThreads), 0, s, xp, np, qp, sp); return true;
      case 2: hipLaunchKernelGGL((quantize_rows_pair_kernel<2>), g2, dim3(kSwapThreads), 0, s, xp, np, qp, sp); return true;
      case 4: hipLaunchKernelGGL((quantize_rows_pair_kernel<4>), g2, dim3(kSwapThreads), 0, s, xp, np, qp, sp); return true;
      case 8: hipLaunchKernelGGL((quantize_rows_pair_kernel<8>), g2, dim3(kSwapThreads), 0, s, xp, np, qp, sp); return true;
      case 16: hipLaunchKernelGGL((quantize_rows_pair_kernel<16>), g2, dim3(kSwapThreads), 0, s, xp, np, qp, sp); return true;
      case 32: hipLaunchKernelGGL((quantize_rows_pair_kernel<32>), g2, dim3(kSwapThreads), 0, s, xp, np, qp, sp); return true;
      default: break;
    }
  }
#define COOPT_RC(GV)                                                                               \
  case GV:                                                                                         \
    if (quant) {                                                                                   \
      if (bits == 8)                                                                               \
        hipLaunchKernelGGL((quantize_rows_kernel<GV, 8>), dim3(grid), dim3(kSwapThreads), 0, s,     \
                           static_cast<const uint16_t*>(x), n, static_cast<unsigned char*>(q),     \
                           static_cast<uint16_t*>(const_cast<void*>(scale)));                      \
      else                                                                                         \
        hipLaunchKernelGGL((quantize_rows_kernel<GV, 4>), dim3(grid), dim3(kSwapThreads), 0, s,     \
                           static_cast<const uint16_t*>(x), n, static_cast<unsigned char*>(q),     \
                           static_cast<uint16_t*>(const_cast<void*>(scale)));                      \
    } else {                                                                                       \
      if (bits == 8)                                                                               \
        hipLaunchKernelGGL((dequantize_rows_kernel<GV, 8>), dim3(grid), dim3(kSwapThreads), 0, s,   \
                           static_cast<const unsigned char*>(q), static_cast<const uint16_t*>(scale), \
                           n, static_cast<uint16_t*>(const_cast<void*>(x)));                       \
      else                                                                                         \
        hipLaunchKernelGGL((dequantize_rows_kernel<GV, 4>), dim3(grid), dim3(kSwapThreads), 0, s,   \
                           static_cast<const unsigned char*>(q), static_cast<const uint16_t*>(scale), \
                           n, static_cast<uint16_t*>(const_cast<void*>(x)));                       \
    }                                                                                              \
    break;
  switch (G) {
    COOPT_RC(1)
    COOPT_RC(2)
    COOPT_RC(4)
    COOPT_RC(8)
    COOPT_RC(16)
    COOPT_RC(32)
    COOPT_RC(64)
    default:
      return false;
  }
#undef COOPT_RC
  return true;
}

template <int BITS, bool I8>
int launch_swap(bool out, int G, const CacheSet& cs, int n, int64_t c_bs, int64_t c_ts, int64_t c_hs,
                int64_t s_bs, int64_t s_ts, int64_t s_hs, const int64_t* ids, int nid,
                int bs, int Hkv, int64_t num_blocks, void* q, void* scale, int64_t q_stride,
                int64_t s_stride, hipStream_t stream) {
  if (nid == 0 || n == 0) return COOPT_OK;
  const int64_t chunks = static_cast<int64_t>(bs) * Hkv * G;  // of one block
  // U chunks per thread (section above); a launch that would then fill fewer than
  // kSwapSmallGrid workgroups (one layer of a short sequence) takes one chunk per thread, as
  // its time is latency, not bandwidth
  int U = out ? kSwapOutU : kSwapInU;
  if (nid * ((chunks + U * kSwapThreads - 1) / (U * kSwapThreads)) * n < kSwapSmallGrid) U = 1;
  const int64_t slabs = (chunks + U * kSwapThreads - 1) / (U * kSwapThreads);
  COOPT_REQUIRE(chunks <= INT32_MAX && static_cast<int64_t>(nid) * slabs <= INT32_MAX,
                "swap too large for one launch");
  if constexpr (BITS == 8 && !I8) {
    // bf16 caches out at 8 bits, launches large enough for U > 1 chunks a thread and 16-byte
    // aligned rows: two chunks a lane (swap_out_pair_kernel)
    if (out && U != 1 && G >= 2 && (reinterpret_cast<uintptr_t>(q) & 15u) == 0) {
      const int64_t sl2 = (chunks / 2 + kSwapPairOutU * kSwapThreads - 1) / (kSwapPairOutU * kSwapThreads);
      const dim3 g2(static_cast<unsigned>(nid * sl2), static_cast<unsigned>(n));
      const int s2 = static_cast<int>(sl2);
      unsigned char* qp = static_cast<unsigned char*>(q);
      uint16_t* sp = static_cast<uint16_t*>(scale);
#define COOPT_SWP(GV)                                                                             \
  case GV:                                                                                        \
    hipLaunchKernelGGL((swap_out_pair_kernel<GV / 2>), g2, dim3(kSwapThreads), 0, stream, cs, c_bs, \
                       c_ts, c_hs, ids, s2, bs, Hkv, num_blocks, qp, sp, q_stride, s_stride);      \
    return coopt::check_launch("coopt_kv_swap_out");
      switch (G) {
        COOPT_SWP(2)
        COOPT_SWP(4)
        COOPT_SWP(8)
        COOPT_SWP(16)
        COOPT_SWP(32)
        COOPT_SWP(64)
        default:
          break;
      }
#undef COOPT_SWP
    }
  }
  const dim3 grid(static_cast<unsigned>(nid * slabs), static_cast<unsigned>(n));
  const int sl = static_cast<int>(slabs);
#define COOPT_SW_U(GV, UO, UI)                                                                    \
  if (out)                                                                                        \
    hipLaunchKernelGGL((swap_out_kernel<GV, BITS, I8, UO>), grid, dim3(kSwapThreads), 0, stream,  \
                       cs, c_bs, c_ts, c_hs, s_bs, s_ts, s_hs, ids, sl, bs, Hkv, num_blocks,      \
                       static_cast<unsigned char*>(q), static_cast<uint16_t*>(scale), q_stride,   \
                       s_stride);                                                                 \
  else                                                                                            \
    hipLaunchKernelGGL((swap_in_kernel<GV, BITS, I8, UI>), grid, dim3(kSwapThreads), 0, stream,   \
                       static_cast<const unsigned char*>(q), static_cast<const uint16_t*>(scale), \
                       q_stride, s_stride, ids, sl, bs, Hkv, num_blocks, cs, c_bs, c_ts, c_hs,    \
                       s_bs, s_ts, s_hs);
#define COOPT_SW(GV)                                  \
  case GV:                                            \
    if (U == 1) {                                     \
      COOPT_SW_U(GV, 1, 1)                            \
    } else {                                          \
      COOPT_SW_U(GV, kSwapOutU, kSwapInU)             \
    }                                                 \
    break;
  switch (G) {
    COOPT_SW(1)
    COOPT_SW(2)
    COOPT_SW(4)
    COOPT_SW(8)
    COOPT_SW(16)
    COOPT_SW(32)
    COOPT_SW(64)
    default:
      return COOPT_EINVAL;
  }
#undef COOPT_SW_U
#undef COOPT_SW
  return coopt::check_launch(out ? "coopt_kv_swap_out" : "coopt_kv_swap_in");
}

// Argument checks shared by swap_out / swap_in; returns COOPT_OK or an error code.
int check_swap(int bits, int cache_dtype, const void* cache, int64_t c_bs, int64_t c_ts,
               int64_t c_hs, const void* cscale, const int64_t* ids, int nid, int bs, int Hkv,
               int D, int64_t num_blocks, const void* q, const void* scale) {
  COOPT_REQUIRE(bits == 16 || bits == 8 || bits == 4, "bits must be 16, 8 or 4");
  COOPT_REQUIRE(cache_dtype == COOPT_DT_BF16 || cache_dtype == COOPT_DT_I8,
                "cache_dtype must be COOPT_DT_BF16 or COOPT_DT_I8");
  COOPT_REQUIRE(cache_dtype == COOPT_DT_BF16 || bits == 8, "an INT8 cache swaps at 8 bits");
  COOPT_REQUIRE(nid >= 0 && bs > 0 && Hkv > 0 && num_blocks > 0, "bad sizes");
  COOPT_REQUIRE(D % 8 == 0 && D >= 8 && D <= 512 && ((D / 8) & (D / 8 - 1)) == 0,
                "D must be 8 * a power of two, at most 512");
  if (nid == 0) return COOPT_OK;
  COOPT_REQUIRE(cache && ids && q && (bits == 16 || scale), "null pointer");
  const int qalign = bits == 16 ? 16 : (bits == 8 ? 8 : 4);
  COOPT_REQUIRE((reinterpret_cast<uintptr_t>(q) % qalign) == 0, "swap buffer misaligned");
  if (cache_dtype == COOPT_DT_I8) {
    COOPT_REQUIRE(cscale != nullptr, "INT8 cache needs its scale cache");
    COOPT_REQUIRE((reinterpret_cast<uintptr_t>(cache) & 7u) == 0 && c_bs % 8 == 0 && c_ts % 8 == 0 &&
                      c_hs % 8 == 0, "INT8 cache rows must be 8-byte aligned");
  } else {
    COOPT_REQUIRE(coopt::aligned16(cache) && c_bs % 8 == 0 && c_ts % 8 == 0 && c_hs % 8 == 0,
                  "bf16 cache rows must be 16-byte aligned");
  }
  return COOPT_OK;
}

int dispatch_swap(bool out, int bits, int cache_dtype, const CacheSet& cs, int n, int64_t c_bs,
                  int64_t c_ts, int64_t c_hs, int64_t s_bs, int64_t s_ts, int64_t s_hs,
                  const int64_t* ids, int nid, int bs, int Hkv, int D, int64_t num_blocks, void* q,
                  void* scale, int64_t q_stride, int64_t s_stride, hipStream_t s) {
  const int G = D / 8;
  if (cache_dtype == COOPT_DT_I8)
    return launch_swap<8, true>(out, G, cs, n, c_bs, c_ts, c_hs, s_bs, s_ts, s_hs, ids, nid, bs, Hkv,
                                num_blocks, q, scale, q_stride, s_stride, s);
  if (bits == 16)
    return launch_swap<16, false>(out, G, cs, n, c_bs, c_ts, c_hs, s_bs, s_ts, s_hs, ids, nid, bs, Hkv,
                                  num_blocks, q, scale, q_stride, s_stride, s);
  if (bits == 8)
    return launch_swap<8, false>(out, G, cs, n, c_bs, c_ts, c_hs, s_bs, s_ts, s_hs, ids, nid, bs, Hkv,
                                 num_blocks, q, scale, q_stride, s_stride, s);
  return launch_swap<4, false>(out, G, cs, n, c_bs, c_ts, c_hs, s_bs, s_ts, s_hs, ids, nid, bs, Hkv,
                               num_blocks, q, scale, q_stride, s_stride, s);
}

// Swapped bytes of one cache's rows (codes; scales are nid * bs * Hkv fp16).
int64_t swap_q_bytes(int bits, int nid, int bs, int Hkv, int D) {
  return static_cast<int64_t>(nid) * bs * Hkv * (D / 8) * (bits == 16 ? 16 : (bits == 8 ? 8 : 4));
}

// n caches in launches of up to kMaxSwapCaches; caches[i] (and scales[i]) swap with the
// rows at q + i * swap_q_bytes and scale + i * nid * bs * Hkv.
int swap_caches(bool out, int bits, int cache_dtype, int n, const void* const* caches,
                const void* const* scales, int64_t c_bs, int64_t c_ts, int64_t c_hs, int64_t s_bs,
                int64_t s_ts, int64_t s_hs, const int64_t* ids, int nid, int bs, int Hkv, int D,
                int64_t num_blocks, void* q, void* scale, hipStream_t s) {
  const int64_t qb = swap_q_bytes(bits, nid, bs, Hkv, D);
  const int64_t sb = static_cast<int64_t>(nid) * bs * Hkv;
  for (int i0 = 0; i0 < n; i0 += kMaxSwapCaches) {
    const int m = n - i0 < kMaxSwapCaches ? n - i0 : kMaxSwapCaches;
    CacheSet cs{};
    for (int i = 0; i < m; ++i) {
      cs.c[i] = caches[i0 + i];
      cs.s[i] = scales ? static_cast<uint16_t*>(const_cast<void*>(scales[i0 + i])) : nullptr;
    }
    unsigned char* qc = static_cast<unsigned char*>(q) + i0 * qb;
    uint16_t* sc = scale ? static_cast<uint16_t*>(scale) + i0 * sb : nullptr;
    const int rc = dispatch_swap(out, bits, cache_dtype, cs, m, c_bs, c_ts, c_hs, s_bs, s_ts, s_hs,
                                 ids, nid, bs, Hkv, D, num_blocks, qc, sc, qb, sb, s);
    if (rc != COOPT_OK) return rc;
  }
  return COOPT_OK;
}

}  // namespace

extern "C" int coopt_qkv_epilogue(int cache_dtype, const void* qkv, int64_t qkv_tok_stride,
                                  const float* part, int ks, int64_t slice_stride,
                                  const int64_t* positions, const void* cos, const void* sin,
                                  int64_t table_stride, int max_pos, void* q_out,
                                  int64_t q_tok_stride, int64_t q_head_stride, void* k_cache,
                                  void* v_cache, int64_t c_blk_stride, int64_t c_tok_stride,
                                  int64_t c_head_stride, void* k_scale, void* v_scale,
                                  int64_t s_blk_stride, int64_t s_tok_stride,
                                  int64_t s_head_stride, const int64_t* slot_mapping, int T,
                                  int Hq, int Hkv, int D, int block_size, int64_t num_blocks,
                                  coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(cache_dtype == COOPT_DT_BF16 || cache_dtype == COOPT_DT_I8,
                "cache_dtype must be COOPT_DT_BF16 or COOPT_DT_I8");
  COOPT_REQUIRE(T >= 0 && Hq > 0 && Hkv > 0 && block_size > 0 && num_blocks > 0 && max_pos > 0,
                "bad sizes");
  COOPT_REQUIRE(D == 64 || D == 128 || D == 256, "D must be 64, 128 or 256");
  if (T == 0) return COOPT_OK;
  COOPT_REQUIRE((qkv != nullptr) != (part != nullptr), "give exactly one of qkv and part");
  COOPT_REQUIRE(positions && cos && sin && q_out && k_cache && v_cache && slot_mapping,
                "null pointer");
  if (part) {
    COOPT_REQUIRE(ks >= 1 && ks <= 16, "1 to 16 partial slices");
    COOPT_REQUIRE(coopt::aligned16(part) && slice_stride % 4 == 0 &&
                      slice_stride >= static_cast<int64_t>(T) * (Hq + 2 * Hkv) * D,
                  "partials must be 16-byte aligned [ks, >= T, (Hq + 2 Hkv) D] fp32");
  } else {
    COOPT_REQUIRE(coopt::aligned16(qkv) && qkv_tok_stride % 8 == 0 &&
                      qkv_tok_stride >= static_cast<int64_t>(Hq + 2 * Hkv) * D,
                  "qkv rows must be 16-byte aligned, at least (Hq + 2 Hkv) D wide");
  }
  COOPT_REQUIRE(coopt::aligned16(cos) && coopt::aligned16(sin) && table_stride % 8 == 0 &&
                    table_stride >= D / 2,
                "cos/sin rows must be 16-byte aligned with at least D/2 entries");
  COOPT_REQUIRE(coopt::aligned16(q_out) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0,
                "q_out rows must be 16-byte aligned");
  const bool int8 = cache_dtype == COOPT_DT_I8;
  if (int8) {
    COOPT_REQUIRE(k_scale && v_scale, "INT8 cache needs k_scale and v_scale");
    COOPT_REQUIRE((reinterpret_cast<uintptr_t>(k_cache) & 7u) == 0 &&
                      (reinterpret_cast<uintptr_t>(v_cache) & 7u) == 0 && c_blk_stride % 8 == 0 &&
                      c_tok_stride % 8 == 0 && c_head_stride % 8 == 0,
                  "INT8 cache rows must be 8-byte aligned");
  } else {
    COOPT_REQUIRE(coopt::aligned16(k_cache) && coopt::aligned16(v_cache) &&
                      c_blk_stride % 8 == 0 && c_tok_stride % 8 == 0 && c_head_stride % 8 == 0,
                  "bf16 cache rows must be 16-byte aligned");
  }
  QkvArgs a{static_cast<const uint16_t*>(qkv), qkv_tok_stride, part, ks, slice_stride, positions,
            static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), table_stride,
            max_pos, static_cast<uint16_t*>(q_out), q_tok_stride, q_head_stride, k_cache, v_cache,
            c_blk_stride, c_tok_stride, c_head_stride, static_cast<uint16_t*>(k_scale),
            static_cast<uint16_t*>(v_scale), s_blk_stride, s_tok_stride, s_head_stride,
            slot_mapping, T, Hq, Hkv, D, block_size, num_blocks * block_size,
            (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1};
  const int G = D / 8;
  const int64_t lanes = static_cast<int64_t>(T) * G;
  COOPT_REQUIRE(lanes <= 0x7fffff00LL && Hq + Hkv <= 65535, "T * D / 8 must stay below 2^31");
  const dim3 grid(static_cast<unsigned>((lanes + 255) / 256), static_cast<unsigned>(Hq + Hkv));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // partials with at most 8 slices: the compile-time-bounded loader (all loads up front)
  const int kb = part ? partials_bound(ks) : 0;
  const int kbound = kb <= 8 ? kb : 0;
#define COOPT_QKV_KS(GV, KSV)                                                                   \
  case KSV:                                                                                     \
    if (int8) hipLaunchKernelGGL((qkv_epilogue_kernel<GV, true, KSV>), grid, dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((qkv_epilogue_kernel<GV, false, KSV>), grid, dim3(256), 0, st, a);    \
    break;
#define COOPT_QKV(GV)          \
  case GV:                     \
    switch (kbound) {          \
      COOPT_QKV_KS(GV, 0)      \
      COOPT_QKV_KS(GV, 1)      \
      COOPT_QKV_KS(GV, 2)      \
      COOPT_QKV_KS(GV, 4)      \
      COOPT_QKV_KS(GV, 8)      \
    }                          \
    break;
  switch (G) {
    COOPT_QKV(8)
    COOPT_QKV(16)
    COOPT_QKV(32)
  }
#undef COOPT_QKV
#undef COOPT_QKV_KS
  return coopt::check_launch("coopt_qkv_epilogue");
}

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
  auto s = static_cast<hipStream_t>(stream);
  if (in_dtype == COOPT_DT_BF16 && launch_rows_codec(true, bits, x, rows, D, q, scale, s))
    return coopt::check_launch("coopt_quantize");
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
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
  auto s = static_cast<hipStream_t>(stream);
  if (out_dtype == COOPT_DT_BF16 &&
      launch_rows_codec(false, bits, out, rows, D, const_cast<void*>(q), scale, s))
    return coopt::check_launch("coopt_dequantize");
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
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

extern "C" int coopt_kv_swap_out(int bits, int cache_dtype, const void* cache,
                                 int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                                 const void* cache_scale, int64_t s_blk_stride,
                                 int64_t s_tok_stride, int64_t s_head_stride,
                                 const int64_t* block_ids, int num_ids, int block_size, int Hkv,
                                 int D, int64_t num_blocks, void* q, void* scale,
                                 coopt_stream_t stream) {
  const int rc = check_swap(bits, cache_dtype, cache, c_blk_stride, c_tok_stride, c_head_stride,
                            cache_scale, block_ids, num_ids, block_size, Hkv, D, num_blocks, q, scale);
  if (rc != COOPT_OK || num_ids == 0) return rc;
  coopt::clear_error();
  return swap_caches(true, bits, cache_dtype, 1, &cache, &cache_scale, c_blk_stride, c_tok_stride,
                     c_head_stride, s_blk_stride, s_tok_stride, s_head_stride, block_ids, num_ids,
                     block_size, Hkv, D, num_blocks, q, scale, static_cast<hipStream_t>(stream));
}

extern "C" int coopt_kv_swap_in(int bits, int cache_dtype, const void* q, const void* scale,
                                const int64_t* block_ids, int num_ids, int block_size, int Hkv,
                                int D, int64_t num_blocks, void* cache, int64_t c_blk_stride,
                                int64_t c_tok_stride, int64_t c_head_stride, void* cache_scale,
                                int64_t s_blk_stride, int64_t s_tok_stride, int64_t s_head_stride,
                                coopt_stream_t stream) {
  const int rc = check_swap(bits, cache_dtype, cache, c_blk_stride, c_tok_stride, c_head_stride,
                            cache_scale, block_ids, num_ids, block_size, Hkv, D, num_blocks, q, scale);
  if (rc != COOPT_OK || num_ids == 0) return rc;
  coopt::clear_error();
  const void* c = cache;
  const void* cs = cache_scale;
  return swap_caches(false, bits, cache_dtype, 1, &c, &cs, c_blk_stride, c_tok_stride,
                     c_head_stride, s_blk_stride, s_tok_stride, s_head_stride, block_ids, num_ids,
                     block_size, Hkv, D, num_blocks, const_cast<void*>(q), const_cast<void*>(scale),
                     static_cast<hipStream_t>(stream));
}

extern "C" int coopt_kv_swap_out_caches(int bits, int cache_dtype, int num_caches,
                                        const void* const* caches, const void* const* cache_scales,
                                        int64_t c_blk_stride, int64_t c_tok_stride,
                                        int64_t c_head_stride, int64_t s_blk_stride,
                                        int64_t s_tok_stride, int64_t s_head_stride,
                                        const int64_t* block_ids, int num_ids, int block_size,
                                        int Hkv, int D, int64_t num_blocks, void* q, void* scale,
                                        coopt_stream_t stream) {
  COOPT_REQUIRE(num_caches >= 0 && (num_caches == 0 || caches), "bad cache list");
  for (int i = 0; i < num_caches; ++i) {
    const int rc = check_swap(bits, cache_dtype, caches[i], c_blk_stride, c_tok_stride,
                              c_head_stride, cache_scales ? cache_scales[i] : nullptr, block_ids,
                              num_ids, block_size, Hkv, D, num_blocks, q, scale);
    if (rc != COOPT_OK) return rc;
  }
  if (num_caches == 0 || num_ids == 0) return COOPT_OK;
  coopt::clear_error();
  return swap_caches(true, bits, cache_dtype, num_caches, caches, cache_scales, c_blk_stride,
                     c_tok_stride, c_head_stride, s_blk_stride, s_tok_stride, s_head_stride,
                     block_ids, num_ids, block_size, Hkv, D, num_blocks, q, scale,
                     static_cast<hipStream_t>(stream));
}

extern "C" int coopt_kv_swap_in_caches(int bits, int cache_dtype, int num_caches, const void* q,
                                       const void* scale, const int64_t* block_ids, int num_ids,
                                       int block_size, int Hkv, int D, int64_t num_blocks,
                                       void* const* caches, void* const* cache_scales,
                                       int64_t c_blk_stride, int64_t c_tok_stride,
                                       int64_t c_head_stride, int64_t s_blk_stride,
                                       int64_t s_tok_stride, int64_t s_head_stride,
                                       coopt_stream_t stream) {
  COOPT_REQUIRE(num_caches >= 0 && (num_caches == 0 || caches), "bad cache list");
  for (int i = 0; i < num_caches; ++i) {
    const int rc = check_swap(bits, cache_dtype, caches[i], c_blk_stride, c_tok_stride,
                              c_head_stride, cache_scales ? cache_scales[i] : nullptr, block_ids,
                              num_ids, block_size, Hkv, D, num_blocks, q, scale);
    if (rc != COOPT_OK) return rc;
  }
  if (num_caches == 0 || num_ids == 0) return COOPT_OK;
  coopt::clear_error();
  return swap_caches(false, bits, cache_dtype, num_caches,
                     reinterpret_cast<const void* const*>(caches),
                     reinterpret_cast<const void* const*>(cache_scales),
                     c_blk_stride, c_tok_stride, c_head_stride, s_blk_stride, s_tok_stride,
                     s_head_stride, block_ids, num_ids, block_size, Hkv, D, num_blocks,
                     const_cast<void*>(q), const_cast<void*>(scale),
                     static_cast<hipStream_t>(stream));
}
