// Paged GQA verification attention for gfx950 (replaces flash_attn_varlen_func at
// engine/model.py:244-247 for the speculative-verify shapes: a few query rows per sequence).
//
// Work decomposition.  Grid (context split, KV head, sequence); 256 threads = 4 waves.  All
// G = Hq/Hkv query heads of a KV head and all n query rows of the sequence are packed into
// R = G*n "rows" (row r = head_local * n + j), so each K/V byte is read once per KV head.
// A block covers `split` keys of one (sequence, KV head); its 4 waves take 32-key tiles in
// turn and each keeps its own online softmax; the waves merge through LDS.  With one split
// the block writes the bf16 output; otherwise it writes its (max, sum) and unnormalised fp32
// partial rows to the workspace and a second launch (merge_kernel, one block per (KV head,
// sequence)) combines the splits -- the kernel boundary orders the two, so no block waits on
// another and no cross-workgroup fence is needed.
//
// MFMA layout (v_mfma_f32_16x16x32_bf16, lane l, g = l/16):
//   scores  S^T[key][row] = K[key][:] . Q[row][:]   A = K   (key l%16, 8 d values of group g)
//                                                   B = Q^T (row l%16, the same 8 d values)
//           -> lane l holds row l%16 and keys 4g..4g+3 of each 16-key tile
//   output  O^T[d][row] += V^T[d][keys] . P^T[keys][row]
//           B = P^T: lane l supplies row l%16 and keys {4g..4g+3} of tile 0 and of tile 1,
//           which are exactly the score registers it already holds -- no shuffles.
//           A = V^T: d = l%16, the same 8 keys, read from the LDS copy of the V tile.
//   Every lane's accumulators therefore belong to a single query row, so the online-softmax
//   rescale is a per-lane scalar.
// INT8 KV: every code is dequantised to bf16(float(code) * scale) -- the values the reference
// attends over after dequantize(quantize(KV)) (eval/quality.py:48-52) -- K in registers as it
// is loaded, V before it is staged in LDS, so the MFMA stages are those of the bf16 path and
// the INT8 result equals the bf16 kernel run on the dequantised cache.
#include <math.h>

#include "common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kTileKeys = 32;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const void* kc;
  const void* vc;
  int64_t c_bs, c_ts, c_hs;
  const uint16_t* ks;
  const uint16_t* vs;
  int64_t s_bs, s_ts, s_hs;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* cu;
  const int32_t* seq_lens;
  int G, Hkv, bs_shift;
  int max_seqlen_k;
  int64_t num_blocks;
  float scale_log2;
  uint16_t* out;
  int64_t o_ts, o_hs;
  int split, max_splits, rmax;
  float2* part_ml;
  float* part_o;
};

__device__ __forceinline__ f32x4_t mfma_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// Four int8 codes of one word -> bf16(float(code) * scale), as dequantize(q, s, 8, bf16)
// computes them (engine/kv_tier_manager.py:41): the fp32 product is exact, then one RNE.
__device__ __forceinline__ u32x2_t dequant4(uint32_t w, float sc) {
  const float c0 = static_cast<float>(static_cast<int8_t>(w & 0xff));
  const float c1 = static_cast<float>(static_cast<int8_t>((w >> 8) & 0xff));
  const float c2 = static_cast<float>(static_cast<int8_t>((w >> 16) & 0xff));
  const float c3 = static_cast<float>(static_cast<int8_t>(w >> 24));
  return u32x2_t{pack_bf16x2(c0 * sc, c1 * sc), pack_bf16x2(c2 * sc, c3 * sc)};
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int64_t clamp_page(int32_t page, int64_t num_blocks) {
  return page < 0 ? 0 : (page >= num_blocks ? num_blocks - 1 : page);
}

template <int D, bool INT8>
struct Tile {
  static constexpr int kKs = D / 32;                   // MFMA k-steps over the head dim
  static constexpr int kDt = D / 16;                   // 16-wide d tiles of the output
  static constexpr int kElt = INT8 ? 1 : 2;            // bytes per cached element
  static constexpr int kChunkElems = 16 / kElt;        // elements per 16-byte chunk
  static constexpr int kChunksPerKey = D / kChunkElems;
  static constexpr int kVLoads = kTileKeys * kChunksPerKey / 64;  // 16-byte V loads per lane
  // LDS pitch of one staged (bf16) V row in bytes: padded so the transposed reads of the
  // four key groups land in different banks.
  static constexpr int kPitch = 2 * D + 8;
  static constexpr int kWaveLds = kTileKeys * kPitch;
};

// Up to 32 query rows the kernel fits 2 waves per SIMD; 48-64 rows need the full register
// file (accumulators spill into AGPRs) and run at 1 wave per SIMD.
template <int D, bool INT8, int RT>
__global__ __launch_bounds__(kThreads, (RT <= 2 ? 2 : 1)) void verify_attn_kernel(AttnArgs a) {
  using TL = Tile<D, INT8>;
  constexpr int kRows = RT * 16;
  constexpr int kOPitch = D + 4;  // fp32 row pitch of the merged output in LDS
  constexpr int kStageBytes = kWaves * TL::kWaveLds;
  constexpr int kMergeBytes = kRows * kOPitch * 4;
  constexpr int kLdsBytes = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];
  __shared__ float sm_m[kWaves][kRows];
  __shared__ float sm_l[kWaves][kRows];
  __shared__ float sm_M[kRows];
  __shared__ float sm_L[kRows];

  const int b = blockIdx.z, hkv = blockIdx.y, sidx = blockIdx.x;
  const int q0 = a.cu[b];
  const int n = a.cu[b + 1] - q0;
  // Clamps keep a malformed call (seq_len > max_seqlen_k, q_len > max_seqlen_q, block ids
  // outside the pool) inside its buffers: such calls give wrong rows, never stray accesses.
  const int L = min(a.seq_lens[b], a.max_seqlen_k);
  if (n <= 0) return;
  const int nsplit = L > 0 ? (L + a.split - 1) / a.split : 1;
  if (sidx >= nsplit) return;
  const int R = min(min(a.G * n, kRows), a.rmax);
  const int k_begin = sidx * a.split;
  const int k_end = min(L, k_begin + a.split);

  const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bs_mask = (1 << a.bs_shift) - 1;
  const int32_t* table = a.bt + static_cast<int64_t>(b) * a.bt_stride;

  // ---- Q operand (B of the score MFMA) and per-row causal limits ----
  u32x4_t qreg[RT][TL::kKs];
  int lim[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 16 + l16;
    if (r < R) {
      const int hl = r / n, j = r - hl * n;
      const uint16_t* qp = a.q + static_cast<int64_t>(q0 + j) * a.q_ts +
                           static_cast<int64_t>(hkv * a.G + hl) * a.q_hs + grp * 8;
#pragma unroll
      for (int ks = 0; ks < TL::kKs; ++ks) qreg[rt][ks] = *reinterpret_cast<const u32x4_t*>(qp + ks * 32);
      lim[rt] = L - n + j;  // bottom-right aligned causal mask
    } else {
#pragma unroll
      for (int ks = 0; ks < TL::kKs; ++ks) qreg[rt][ks] = u32x4_t{0, 0, 0, 0};
      lim[rt] = -1;
    }
  }

  f32x4_t o[RT][TL::kDt];
  float m_run[RT], l_run[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < TL::kDt; ++dt) o[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  unsigned char* stage = lds + wave * TL::kWaveLds;
  const int ntiles = (k_end - k_begin + kTileKeys - 1) / kTileKeys;
  const unsigned char* kbase = static_cast<const unsigned char*>(a.kc);
  const unsigned char* vbase = static_cast<const unsigned char*>(a.vc);
  const int64_t head_off = static_cast<int64_t>(hkv) * a.c_hs;
  const int64_t shead_off = static_cast<int64_t>(hkv) * a.s_hs;

  // `wave` is uniform, so the tile loop and the two page lookups per tile are scalar.  A
  // 32-key tile starts on a multiple of 32 and block_size >= 16, so its keys lie in at most
  // two pages: the one holding key kb and the one holding key kb + 16 (keys past the end are
  // clamped to L - 1, which stays in the page of its 16-key half).  The page ids of the
  // wave's next tile are fetched one iteration ahead.
  auto page_of = [&](int key) {
    return clamp_page(table[min(key, L - 1) >> a.bs_shift], a.num_blocks);
  };
  int64_t nxt0 = 0, nxt1 = 0;
  if (wave < ntiles) {
    nxt0 = page_of(k_begin + wave * kTileKeys);
    nxt1 = page_of(k_begin + wave * kTileKeys + 16);
  }
  for (int tile = wave; tile < ntiles; tile += kWaves) {
    const int kb = k_begin + tile * kTileKeys;
    const int64_t pg0 = nxt0, pg1 = nxt1;
    if (tile + kWaves < ntiles) {
      nxt0 = page_of(kb + kWaves * kTileKeys);
      nxt1 = page_of(kb + kWaves * kTileKeys + 16);
    }

    // ---- issue every load of the tile before using any of them ----
    // K operand: lane's key for each 16-key sub-tile, 8 d values per k-step.
    u32x4_t kraw[2][TL::kKs];
    u32x2_t kraw8[2][TL::kKs];
    float ksc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = min(kb + kt * 16 + l16, L - 1);
      const int64_t tok = static_cast<int64_t>(key & bs_mask);
      const int64_t pg = kt ? pg1 : pg0;
      const int64_t row = pg * a.c_bs + tok * a.c_ts + head_off;
#pragma unroll
      for (int ks = 0; ks < TL::kKs; ++ks) {
        const int64_t e = row + ks * 32 + grp * 8;
        if constexpr (INT8) {
          kraw8[kt][ks] = *reinterpret_cast<const u32x2_t*>(kbase + e);
        } else {
          kraw[kt][ks] = *reinterpret_cast<const u32x4_t*>(kbase + 2 * e);
        }
      }
      if constexpr (INT8) ksc[kt] = f16_to_f32(a.ks[pg * a.s_bs + tok * a.s_ts + shead_off]);
    }
    // V tile: coalesced 16-byte chunks, staged through LDS below.
    u32x4_t vreg[TL::kVLoads];
    float vsc[TL::kVLoads];
#pragma unroll
    for (int it = 0; it < TL::kVLoads; ++it) {
      const int id = it * 64 + lane;
      const int kk = id / TL::kChunksPerKey, c = id % TL::kChunksPerKey;
      const int key = min(kb + kk, L - 1);
      const int64_t tok = static_cast<int64_t>(key & bs_mask);
      const int64_t pg = kk < 16 ? pg0 : pg1;
      const int64_t row = pg * a.c_bs + tok * a.c_ts + head_off;
      vreg[it] = *reinterpret_cast<const u32x4_t*>(vbase + TL::kElt * row + c * 16);
      vsc[it] = 0.0f;
      if constexpr (INT8) vsc[it] = f16_to_f32(a.vs[pg * a.s_bs + tok * a.s_ts + shead_off]);
    }
    __builtin_amdgcn_sched_barrier(0);

    // K to bf16 MFMA operands (INT8: dequantised with the lane's key scale).
    u32x4_t kreg[2][TL::kKs];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ks = 0; ks < TL::kKs; ++ks) {
        if constexpr (INT8) {
          const u32x2_t lo = dequant4(kraw8[kt][ks][0], ksc[kt]);
          const u32x2_t hi = dequant4(kraw8[kt][ks][1], ksc[kt]);
          kreg[kt][ks] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        } else {
          kreg[kt][ks] = kraw[kt][ks];
        }
      }

    // ---- scores and online softmax ----
    uint32_t pb[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float sv[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < TL::kKs; ++ks) acc = mfma_bf16(kreg[kt][ks], qreg[rt][ks], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb + kt * 16 + grp * 4 + i;
          const float s = acc[i] * a.scale_log2;
          sv[kt][i] = (key > lim[rt] || key >= k_end) ? -INFINITY : s;
        }
      }
      float tmax = fmaxf(fmaxf(fmaxf(sv[0][0], sv[0][1]), fmaxf(sv[0][2], sv[0][3])),
                         fmaxf(fmaxf(sv[1][0], sv[1][1]), fmaxf(sv[1][2], sv[1][3])));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m_run[rt], tmax);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = exp2_fast(m_run[rt] - m_use);
      float p[2][4], psum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[kt][i] = exp2_fast(sv[kt][i] - m_use);
          psum += p[kt][i];
        }
      l_run[rt] = l_run[rt] * alpha + psum;
      m_run[rt] = m_new;
#pragma unroll
      for (int dt = 0; dt < TL::kDt; ++dt) o[rt][dt] *= alpha;
      pb[rt][0] = pack_bf16x2(p[0][0], p[0][1]);
      pb[rt][1] = pack_bf16x2(p[0][2], p[0][3]);
      pb[rt][2] = pack_bf16x2(p[1][0], p[1][1]);
      pb[rt][3] = pack_bf16x2(p[1][2], p[1][3]);
    }

    // ---- stage V in LDS (this wave's region; only this wave reads it) ----
#pragma unroll
    for (int it = 0; it < TL::kVLoads; ++it) {
      const int id = it * 64 + lane;
      const int kk = id / TL::kChunksPerKey, c = id % TL::kChunksPerKey;
      unsigned char* dst = stage + kk * TL::kPitch + c * 2 * TL::kChunkElems;
      if constexpr (INT8) {
        u32x2_t* d64 = reinterpret_cast<u32x2_t*>(dst);
#pragma unroll
        for (int w = 0; w < 4; ++w) d64[w] = dequant4(vreg[it][w], vsc[it]);
      } else {
        u32x2_t* d64 = reinterpret_cast<u32x2_t*>(dst);
        d64[0] = u32x2_t{vreg[it][0], vreg[it][1]};
        d64[1] = u32x2_t{vreg[it][2], vreg[it][3]};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- O^T += V^T . P^T ----
#pragma unroll
    for (int dt = 0; dt < TL::kDt; ++dt) {
      const int d = dt * 16 + l16;
      u32x4_t va;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        uint32_t half[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int e = e2 * 2 + h;
          const int kk = e < 4 ? grp * 4 + e : 16 + grp * 4 + (e - 4);
          half[h] = *reinterpret_cast<const uint16_t*>(stage + kk * TL::kPitch + 2 * d);
        }
        va[e2] = half[0] | (half[1] << 16);
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const u32x4_t pbv = {pb[rt][0], pb[rt][1], pb[rt][2], pb[rt][3]};
        o[rt][dt] = mfma_bf16(va, pbv, o[rt][dt]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the 4 waves ----
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    l_run[rt] += __shfl_xor(l_run[rt], 16, 64);
    l_run[rt] += __shfl_xor(l_run[rt], 32, 64);
    if (grp == 0) {
      sm_m[wave][rt * 16 + l16] = m_run[rt];
      sm_l[wave][rt * 16 + l16] = l_run[rt];
    }
  }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 16 + l16;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][r]);
    float Lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      if (sm_m[w][r] > -INFINITY) Lsum += sm_l[w][r] * exp2_fast(sm_m[w][r] - M);
    const float f = m_run[rt] > -INFINITY ? exp2_fast(m_run[rt] - M) : 0.0f;
#pragma unroll
    for (int dt = 0; dt < TL::kDt; ++dt) o[rt][dt] *= f;
    if (wave == 0 && grp == 0) {
      sm_M[r] = M;
      sm_L[r] = Lsum;
    }
  }
  float* osh = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int r = rt * 16 + l16;
#pragma unroll
        for (int dt = 0; dt < TL::kDt; ++dt) {
          f32x4_t* dst = reinterpret_cast<f32x4_t*>(osh + r * kOPitch + dt * 16 + grp * 4);
          if (w == 0) {
            *dst = o[rt][dt];
          } else {
            *dst = *dst + o[rt][dt];
          }
        }
      }
    }
    __syncthreads();
  }

  constexpr int kCh = D / 8;  // 8-element chunks per row
  const int64_t item = static_cast<int64_t>(b) * a.Hkv + hkv;
  if (nsplit == 1) {
    for (int idx = tid; idx < R * kCh; idx += kThreads) {
      const int r = idx / kCh, c = idx % kCh;
      const float Lr = sm_L[r];
      const float inv = Lr > 0.0f ? 1.0f / Lr : 0.0f;
      const float* src = osh + r * kOPitch + c * 8;
      u32x4_t v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = pack_bf16x2(src[2 * e] * inv, src[2 * e + 1] * inv);
      const int hl = r / n, j = r - hl * n;
      uint16_t* dst = a.out + static_cast<int64_t>(q0 + j) * a.o_ts +
                      static_cast<int64_t>(hkv * a.G + hl) * a.o_hs + c * 8;
      *reinterpret_cast<u32x4_t*>(dst) = v;
    }
    return;
  }

  // ---- several splits: publish this split's partial; merge_kernel combines them ----
  const int64_t pbase = (item * a.max_splits + sidx) * a.rmax;
  for (int idx = tid; idx < R * kCh; idx += kThreads) {
    const int r = idx / kCh, c = idx % kCh;
    const float* src = osh + r * kOPitch + c * 8;
    float* dst = a.part_o + (pbase + r) * D + c * 8;
    reinterpret_cast<f32x4_t*>(dst)[0] = f32x4_t{src[0], src[1], src[2], src[3]};
    reinterpret_cast<f32x4_t*>(dst)[1] = f32x4_t{src[4], src[5], src[6], src[7]};
  }
  if (tid < R) a.part_ml[pbase + tid] = make_float2(sm_M[tid], sm_L[tid]);
}

// Second launch: combines the split partials of every (sequence, KV head) that needed more
// than one split.  Stream order makes the first launch's stores visible here; no fences or
// counters are involved (an agent-scope fence per block writes back and invalidates the L2
// of this multi-XCD part and costs far more than the extra launch).
template <int D>
__global__ __launch_bounds__(kThreads) void merge_kernel(AttnArgs a) {
  const int b = blockIdx.y, hkv = blockIdx.x;
  const int q0 = a.cu[b];
  const int n = a.cu[b + 1] - q0;
  const int L = min(a.seq_lens[b], a.max_seqlen_k);
  if (n <= 0) return;
  const int nsplit = L > 0 ? (L + a.split - 1) / a.split : 1;
  if (nsplit <= 1) return;
  const int R = min(a.G * n, a.rmax);
  constexpr int kCh = D / 8;
  const int64_t ibase = (static_cast<int64_t>(b) * a.Hkv + hkv) * a.max_splits * a.rmax;
  for (int idx = threadIdx.x; idx < R * kCh; idx += kThreads) {
    const int r = idx / kCh, c = idx % kCh;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.part_ml[ibase + s * a.rmax + r].x);
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float Lsum = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
      const float2 ml = a.part_ml[ibase + s * a.rmax + r];
      if (!(ml.x > -INFINITY)) continue;
      const float w = exp2_fast(ml.x - M);
      Lsum += ml.y * w;
      const f32x4_t* src = reinterpret_cast<const f32x4_t*>(a.part_o + (ibase + s * a.rmax + r) * D + c * 8);
      acc0 += src[0] * w;
      acc1 += src[1] * w;
    }
    const float inv = Lsum > 0.0f ? 1.0f / Lsum : 0.0f;
    const u32x4_t v = {pack_bf16x2(acc0[0] * inv, acc0[1] * inv), pack_bf16x2(acc0[2] * inv, acc0[3] * inv),
                       pack_bf16x2(acc1[0] * inv, acc1[1] * inv), pack_bf16x2(acc1[2] * inv, acc1[3] * inv)};
    const int hl = r / n, j = r - hl * n;
    uint16_t* dst = a.out + static_cast<int64_t>(q0 + j) * a.o_ts +
                    static_cast<int64_t>(hkv * a.G + hl) * a.o_hs + c * 8;
    *reinterpret_cast<u32x4_t*>(dst) = v;
  }
}

// Keys per split: a pure function of the launch shape, so the workspace can be sized without
// reading seq_lens.  Aims at ~2048 blocks (8 per CU) for the longest context.
int choose_split(int B, int Hkv, int max_seqlen_k) {
  const int64_t items = static_cast<int64_t>(B) * Hkv;
  int64_t per = (static_cast<int64_t>(max_seqlen_k) * items + 2047) / 2048;
  per = ((per + 127) / 128) * 128;
  if (per < 256) per = 256;
  if (per > 8192) per = 8192;
  return static_cast<int>(per);
}

struct AttnWs {
  size_t ml_off, o_off, total;
};

AttnWs attn_ws_layout(int B, int Hkv, int D, int rmax, int max_splits) {
  auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  AttnWs w;
  const size_t items = static_cast<size_t>(B) * Hkv;
  w.ml_off = 0;
  w.o_off = w.ml_off + al(items * max_splits * rmax * sizeof(float2));
  w.total = w.o_off + al(items * max_splits * rmax * static_cast<size_t>(D) * sizeof(float));
  return w;
}

template <int D, bool INT8>
int launch_rt(int RT, const AttnArgs& a, dim3 grid, hipStream_t s) {
  switch (RT) {
    case 1: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 1>), grid, dim3(kThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 2>), grid, dim3(kThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 3>), grid, dim3(kThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 4>), grid, dim3(kThreads), 0, s, a); break;
    default: return COOPT_EINVAL;
  }
  int rc = coopt::check_launch("coopt_verify_attention");
  if (rc != COOPT_OK || a.max_splits <= 1) return rc;
  hipLaunchKernelGGL((merge_kernel<D>), dim3(grid.y, grid.z), dim3(kThreads), 0, s, a);
  return coopt::check_launch("coopt_verify_attention/merge");
}

}  // namespace

extern "C" size_t coopt_verify_attention_workspace(int B, int Hq, int Hkv, int D, int max_seqlen_q,
                                                   int max_seqlen_k) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || max_seqlen_q <= 0 || max_seqlen_k <= 0) return 0;
  const int rmax = (Hq / Hkv) * max_seqlen_q;
  const int split = choose_split(B, Hkv, max_seqlen_k);
  const int max_splits = (max_seqlen_k + split - 1) / split;
  return attn_ws_layout(B, Hkv, D, rmax, max_splits).total;
}

extern "C" int coopt_verify_attention(int kv_dtype, const void* q, int64_t q_tok_stride,
                                      int64_t q_head_stride, const void* k_cache,
                                      const void* v_cache, int64_t c_blk_stride,
                                      int64_t c_tok_stride, int64_t c_head_stride,
                                      const void* k_scale, const void* v_scale,
                                      int64_t s_blk_stride, int64_t s_tok_stride,
                                      int64_t s_head_stride, const int32_t* block_table,
                                      int64_t bt_stride, const int32_t* cu_seqlens_q,
                                      const int32_t* seq_lens, int B, int Hq, int Hkv, int D,
                                      int block_size, int64_t num_blocks, int max_seqlen_q,
                                      int max_seqlen_k, float softmax_scale, void* out,
                                      int64_t o_tok_stride, int64_t o_head_stride,
                                      void* workspace, size_t workspace_bytes,
                                      coopt_stream_t stream) {
  COOPT_REQUIRE(kv_dtype == COOPT_DT_BF16 || kv_dtype == COOPT_DT_I8,
                "kv_dtype must be COOPT_DT_BF16 or COOPT_DT_I8");
  COOPT_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "Hq must be a multiple of Hkv");
  COOPT_REQUIRE(D == 64 || D == 128, "head_dim must be 64 or 128");
  COOPT_REQUIRE(block_size >= 16 && (block_size & (block_size - 1)) == 0,
                "block_size must be a power of two >= 16");
  COOPT_REQUIRE(max_seqlen_q > 0 && max_seqlen_k > 0, "max_seqlen_q/k must be positive");
  const int G = Hq / Hkv;
  COOPT_REQUIRE(G * max_seqlen_q <= 64, "(Hq/Hkv) * max_seqlen_q must be <= 64");
  COOPT_REQUIRE(bt_stride >= (max_seqlen_k + block_size - 1) / block_size,
                "block_table narrower than ceil(max_seqlen_k / block_size)");
  if (B == 0) return COOPT_OK;
  COOPT_REQUIRE(q && k_cache && v_cache && block_table && cu_seqlens_q && seq_lens && out,
                "null pointer");
  COOPT_REQUIRE(coopt::aligned16(q) && coopt::aligned16(out) && q_tok_stride % 8 == 0 &&
                    q_head_stride % 8 == 0 && o_tok_stride % 8 == 0 && o_head_stride % 8 == 0,
                "q/out rows must be 16-byte aligned");
  const bool int8 = kv_dtype == COOPT_DT_I8;
  if (int8) {
    COOPT_REQUIRE(k_scale && v_scale, "INT8 KV needs k_scale and v_scale");
    COOPT_REQUIRE(coopt::aligned16(k_cache) && coopt::aligned16(v_cache) && c_blk_stride % 16 == 0 &&
                      c_tok_stride % 16 == 0 && c_head_stride % 16 == 0,
                  "INT8 cache rows must be 16-byte aligned");
  } else {
    COOPT_REQUIRE(coopt::aligned16(k_cache) && coopt::aligned16(v_cache) && c_blk_stride % 8 == 0 &&
                      c_tok_stride % 8 == 0 && c_head_stride % 8 == 0,
                  "bf16 cache rows must be 16-byte aligned");
  }
  const size_t need = coopt_verify_attention_workspace(B, Hq, Hkv, D, max_seqlen_q, max_seqlen_k);
  if (workspace_bytes < need || workspace == nullptr) {
    coopt::set_error("coopt_verify_attention: workspace too small");
    return COOPT_EWORKSPACE;
  }
  COOPT_REQUIRE(num_blocks > 0, "num_blocks must be positive");
  coopt::clear_error();

  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_ts = q_tok_stride;
  a.q_hs = q_head_stride;
  a.kc = k_cache;
  a.vc = v_cache;
  a.c_bs = c_blk_stride;
  a.c_ts = c_tok_stride;
  a.c_hs = c_head_stride;
  a.ks = static_cast<const uint16_t*>(k_scale);
  a.vs = static_cast<const uint16_t*>(v_scale);
  a.s_bs = s_blk_stride;
  a.s_ts = s_tok_stride;
  a.s_hs = s_head_stride;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.cu = cu_seqlens_q;
  a.seq_lens = seq_lens;
  a.G = G;
  a.Hkv = Hkv;
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  a.bs_shift = shift;
  a.max_seqlen_k = max_seqlen_k;
  a.num_blocks = num_blocks;
  a.scale_log2 = softmax_scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.o_ts = o_tok_stride;
  a.o_hs = o_head_stride;
  a.split = choose_split(B, Hkv, max_seqlen_k);
  a.max_splits = (max_seqlen_k + a.split - 1) / a.split;
  a.rmax = G * max_seqlen_q;
  const AttnWs w = attn_ws_layout(B, Hkv, D, a.rmax, a.max_splits);
  char* base = static_cast<char*>(workspace);
  a.part_ml = reinterpret_cast<float2*>(base + w.ml_off);
  a.part_o = reinterpret_cast<float*>(base + w.o_off);

  const int RT = (a.rmax + 15) / 16;
  const dim3 grid(a.max_splits, Hkv, B);
  auto s = static_cast<hipStream_t>(stream);
  if (D == 128) return int8 ? launch_rt<128, true>(RT, a, grid, s) : launch_rt<128, false>(RT, a, grid, s);
  return int8 ? launch_rt<64, true>(RT, a, grid, s) : launch_rt<64, false>(RT, a, grid, s);
}
