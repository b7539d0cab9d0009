// Paged GQA verification attention for gfx950 (replaces flash_attn_varlen_func at
// engine/model.py:244-247 for the speculative-verify shapes: a few query rows per sequence).
//
// Work decomposition.  Grid (context split, KV head, sequence); 8 waves per block (4 at 64
// rows).  All G = Hq/Hkv query heads of a KV head and all n query rows of the sequence are
// packed into R = G*n "rows" (row r = head_local * n + j), so each K/V byte is read once per
// KV head.  A block covers `split` keys of one (sequence, KV head); its waves take 32-key
// tiles in turn, each with its own online softmax, and double-buffer them: the loads of a
// wave's next tile are in flight while it computes the current one.  The first tile's loads
// are issued before Q is staged in LDS, and its page lookups before seq_lens is known, so
// the block's start-up round trips overlap.  The waves merge through LDS, each into its own
// region in one round, summed while the output is written.  With one split the block writes
// the bf16 output; otherwise it writes its (max, sum) and unnormalised fp32 rows to the
// workspace and a second launch (merge_kernel, one block per (KV head, sequence)) combines
// the splits -- the kernel boundary orders the two, so no block waits on another and no
// cross-workgroup fence is needed.  A ragged batch with more (sequence, KV head) items than
// one round of blocks holds runs on a 1-D grid whose blocks rank the sequences by length and
// take the items longest first (plan_item), so its long sequences do not start last.
// Items of more than 64 rows (prefill chunks of a mixed batch) are cut into query windows of
// 64/G query rows -- each window is itself a sequence of those rows over the keys its last
// row sees -- and run one unsplit block per (window, KV head): correct at any length.
//
// MFMA layout (v_mfma_f32_16x16x32_{bf16,f16}; lane l, g = l/16, m = l%16):
//   scores  S^T[key][row] = sum_d K[key][d] Q[row][d]     A = K, B = Q^T
//           K is read with 16-byte loads; load c of lane (key m, group g) covers bytes
//           [64c + 16g, +16) of the key row, so one load instruction reads 64 contiguous bytes
//           of each of 16 rows.  The contraction index of k-step ks, element e is therefore
//           d = 32*ks + 8g + e for bf16 and d = 64*(ks/2) + 16g + 8*(ks%2) + e for INT8; the Q
//           operand (staged in LDS) uses the same map.  The result gives lane l row m and
//           keys 4g..4g+3 of each 16-key sub-tile.
//   output  O^T[d][row] += sum_key V[key][d] P[row][key]  A = V^T, B = P^T
//           B = P^T is exactly the score registers (keys 4g..4g+3 of sub-tiles 0 and 1), so P
//           never leaves registers.  A's row index m of d-tile dt stands for d = m*(D/16) + dt,
//           so a lane reads D/16 contiguous elements of each of its 8 keys (whole key rows per
//           16 lanes: coalesced) and the transpose to "8 keys of one d" is a byte select in
//           registers (v_perm / v_cvt_f32_ubyte) -- no LDS staging.  Lane l's accumulators
//           hold row m and d = (4g + i)*(D/16) + dt.
// INT8 KV.  K: every code is dequantised to bf16(float(code) * scale) -- the value
// dequantize() returns (engine/kv_tier_manager.py:41), which the reference attends over --
// as (1024 + code + 128) * s - 1152 * s in one mixed-precision fma on the fp16 word a byte
// select builds (as for V below), exact before the single bf16 rounding, so the score MFMAs
// see the reference's operands.  (Exact codes against a per-row-scaled fp16 Q, with the key
// scale applied to the scores, would save the per-element multiply, but the reference's
// bf16 rounding of K then goes missing: with config 4's x20 outliers the scores reach
// ~200 and the outputs move by up to 5%.)  V: the codes enter the PV MFMAs
// (v_mfma_f32_16x16x32_f16) as exact fp16 integers -- two byte selects place (code + 128)
// under a 0x64 exponent byte, giving 1024 + code + 128 exactly, and one packed fp16 add
// removes the 1152 -- and each key's V scale is folded into its probability,
// fp16(p * s_v * 2^-e_v).  That replaces bf16(p) * bf16(code * s_v) by one fp16 rounding of
// the product (11 bits against two 8-bit roundings) at a third of the VALU work per V
// element.  e_v is a per-wave power-of-two reference that keeps the fp16 product inside
// [2^-14, 2^15] for every scale the fp16 scale cache can hold (up to 65504, i.e. |V| up to
// 8.3e6): it is set from the largest V scale seen so far and enters the softmax exponent, so
// it cancels in o / l like the running max does.
#include <math.h>

#include "common.h"
#include "kv_store.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;  // merge kernel

// Waves per attention block: 8 (one block per CU at two waves per SIMD, i.e. at most 256
// registers per lane) while the accumulators and two tile buffers fit that (RT <= 3), else 4.
constexpr int waves_for(int RT) { return RT <= 3 ? 8 : 4; }
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
  int B;
  int plan;  // blocks order the items longest first (plan_item)
  // Query windows (nwin > 0): a sequence's rows are taken qwin at a time, window w being rows
  // [w * qwin, (w + 1) * qwin) with the keys its last row sees -- on its own a sequence of
  // those rows, so the bottom-right causal mask stays exact.  1-D grid, block x = ((b * nwin)
  // + w) * Hkv + hkv, one split per window.
  int qwin, nwin;
  // Fused qkv epilogue (coopt_verify_attention_qkv): qkv_mode 0 = q is given; 1 = bf16 qkv
  // projection rows; 2 = their fp32 split-K partials.  The block computes its own q rows
  // (RoPE'd, straight into LDS) and writes its KV head's new K/V to the cache first.
  // The cache writes go through kc / vc / ks / vs (the same caches the kernel reads).
  int qkv_mode;
  const void* qkv_src;  // bf16 rows (mode 1) or fp32 partials (mode 2)
  int64_t qkv_stride;   // mode 1: row stride (elements); mode 2: slice stride (floats)
  int qkv_ks;           // mode 2: slices
  const int64_t* pos;
  const uint16_t* cos;
  const uint16_t* sin;
  int tab_stride;
  int max_pos;
  const int64_t* slots;
};

// verify_attn_kernel's leading scalar arguments: the fields its first load round needs (row
// range, key count, the first tile's pages) and the launch mode (0 a grid of (split, KV head,
// sequence), 1 ordered items (plan), 2 query windows).  As scalars ahead of the AttnArgs they are
// preloaded into SGPRs (the build's kernarg-preload option), so that round does not wait for a
// kernel-argument load; the rest of AttnArgs loads alongside it.
#define ATTN_LEAD(a) (a).cu, (a).seq_lens, (a).bt, (a).bt_stride, (a).split, (a).bs_shift, \
                     ((a).plan ? 1 : ((a).nwin > 0 ? 2 : 0))

// Partials of a fused epilogue are reduced with a compile-time slice bound (every load
// unconditional, see Partials4); launches with more slices are rejected on the host.
constexpr int kQkvMaxSlices = 4;

// Batches of up to kPlanSeqs sequences can be ordered by the blocks themselves (one wave,
// one lane per sequence); larger ones run in grid order.
constexpr int kPlanSeqs = 64;

__device__ __forceinline__ f32x4_t mfma_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4_t mfma_f16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Two fp32 -> packed fp16x2, round to nearest even.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), f16x2_t));
}

// Two (code + 128) bytes already placed as the low bytes of two fp16 words whose high bytes
// are 0x64 -> the fp16 pair (code, code): 1024 + u is exact in fp16, and so is u - 128.
__device__ __forceinline__ uint32_t codes_f16x2(uint32_t biased) {
  const f16x2_t v = __builtin_bit_cast(f16x2_t, biased) + f16x2_t{-1152.0f16, -1152.0f16};
  return __builtin_bit_cast(uint32_t, v);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Per-half unsigned max of two words of two u16 each (v_pk_max_u16).
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a),
                                                                __builtin_bit_cast(u16x2_t, b)));
}

// Two fp16 (1024 + code + 128), as codes_f16x2 takes them -> bf16x2 of code * s, rounded
// once: (1024 + u) * s - 1152 * s is code * s exactly (at most 19 significant bits), so each
// fma (one v_fma_mix, the fp16 half read in place) returns it unrounded.
__device__ __forceinline__ uint32_t dequant_pair(uint32_t biased, float s, float sb) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, biased);
  return pack_bf16x2(fmaf(static_cast<float>(h[0]), s, sb), fmaf(static_cast<float>(h[1]), s, sb));
}

__device__ __forceinline__ int64_t clamp_page(int32_t page, int64_t num_blocks) {
  return page < 0 ? 0 : (page >= num_blocks ? num_blocks - 1 : page);
}

// Raw data of one wave's 32-key tile (see the layout notes at the top of the file).
template <int D, bool INT8>
struct RawTile {
  static constexpr int kElt = INT8 ? 1 : 2;
  static constexpr int kKVec = (D / 4) * kElt / 16;  // 16-byte K loads per 16-key sub-tile
  static constexpr int kVWords = (D / 16) * kElt / 4;  // dwords of V per key
  u32x4_t k[2][kKVec];
  uint32_t v[8][kVWords];
  uint32_t ks[2];        // INT8: fp16 scale of the lane's K key (l16) of each sub-tile
  u32x2_t vs[2];         // INT8: fp16 scales of the lane's V keys 4g..4g+3 of each sub-tile
};

// A lane's V words of one key.  The 8- and 16-byte forms (16 lanes: one whole 128- or 256-byte
// key row) are nontemporal loads: V is read once per call, and on MI355X the streaming hint
// raised the rate at every measured shape (bf16 ctx 8192 189 -> 172 us, INT8 107 -> 103 us,
// ragged config 3 70.5 -> 67.4 us).  K keeps plain loads: one K load instruction covers half
// of each of its 16 rows' 128-byte lines, and with the hint config 3 went to 77 us.  The
// 4-byte form (INT8 at D 64, also half a line per instruction) stays plain, unmeasured.
template <int N>
__device__ __forceinline__ void load_words(const unsigned char* p, uint32_t* dst) {
  if constexpr (N == 4) {
    const u32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    dst[0] = x[0]; dst[1] = x[1]; dst[2] = x[2]; dst[3] = x[3];
  } else if constexpr (N == 2) {
    const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    dst[0] = x[0]; dst[1] = x[1];
  } else {
    dst[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

// The item of block blockIdx.x in an ordered launch (one wave, lane t = sequence t, B <=
// kPlanSeqs): sequences are ranked by key count, longest first (ties by index, sequences
// without query rows last), and block k takes KV head k % Hkv of the sequence of rank
// k / Hkv.  With more items than one round of blocks holds, the dispatcher then starts the
// longest and gives CUs that free up the next longest: longest-processing-time-first list
// scheduling, instead of whatever order the batch came in.  out = {sequence, q0, n, L}, the
// values the lane loaded, so the block does not load them again.
__device__ void plan_item(const AttnArgs& a, int lane, int* out) {
  const int t = lane;
  int q0 = 0, n = 0, L = 0, key = -2;
  if (t < a.B) {
    q0 = a.cu[t];
    n = a.cu[t + 1] - q0;
    L = min(a.seq_lens[t], a.max_seqlen_k);
    key = n > 0 ? max(L, 0) : -1;
  }
  // rank by lane reads into scalar registers: B short scalar steps, no LDS round trips
  int rank = 0;
  for (int j = 0; j < a.B; ++j) {
    const int kj = __builtin_amdgcn_readlane(key, j);
    rank += (kj > key || (kj == key && j < t)) ? 1 : 0;
  }
  if (t < a.B && rank == static_cast<int>(blockIdx.x) / a.Hkv) {
    out[0] = t;
    out[1] = q0;
    out[2] = n;
    out[3] = L;
  }
}

// RT row tiles of 16; SC: the scale caches hold consecutive tokens contiguously (token
// stride 1), so a lane's four scales of a sub-tile are one 8-byte load; DB: double-buffer
// the wave's tiles in registers (RT <= 2, and RT 3 with the smaller INT8 tiles; the other
// shapes need the registers for accumulators).
// FUSED: the block runs the qkv epilogue of its rows first, from bf16 rows (1) or split-K
// partials (2) -- a.qkv_mode, fixed at compile time so the epilogue's loads all issue at once
// (a run-time choice of input made the compiler wait for every earlier load where the two
// input paths joined).
template <int D, bool INT8, int RT, bool SC, int FUSED>
__global__ __launch_bounds__(64 * waves_for(RT), 1) void verify_attn_kernel(
    const int32_t* cu_p, const int32_t* sl_p, const int32_t* bt_p, int64_t bt_stride, int split,
    int bs_shift, int mode, AttnArgs a) {
  using Raw = RawTile<D, INT8>;
  constexpr int kWaves = waves_for(RT);
  constexpr int kBlock = 64 * kWaves;
  constexpr bool DB = RT <= 2 || (INT8 && RT == 3);
  constexpr int kKs = D / 32;   // k-steps of the score MFMA
  constexpr int kDt = D / 16;   // d-tiles of the output = V elements per lane per key
  constexpr int kElt = Raw::kElt;
  constexpr int kRows = RT * 16;
  constexpr int kOPitch = D + 4;       // fp32 row pitch of the merged output in LDS
  constexpr int kQPitch = D * 2 + 16;  // byte pitch of a staged Q row (16 rows -> distinct banks)
  constexpr int kQBytes = kRows * kQPitch;
  // The waves merge through kRegions LDS regions of kRows x kOPitch fp32: one per wave when
  // they fit in 144 KB (up to 32 rows at D = 128), else one per two waves.
  constexpr int kRegionFloats = kRows * kOPitch;
  constexpr int kLdsBudget = 144 * 1024;
  constexpr int kRegions = kWaves * kRegionFloats * 4 <= kLdsBudget ? kWaves
                           : ((kWaves / 2) * kRegionFloats * 4 <= kLdsBudget ? kWaves / 2 : 1);
  constexpr int kOBytes = kRegions * kRegionFloats * 4;
  // kOwn: every wave has a region of its own and Q sits beside the regions (within the 160 KB
  // of a CU), so a wave stores its accumulators the moment its last tile is done and one
  // barrier precedes the output pass, which weights each region by 2^(m_w - M) as it sums.
  // Otherwise Q shares the space with the regions and the merge rescales before it stores.
  constexpr bool kOwn = kRegions == kWaves && kOBytes + kQBytes <= 150 * 1024;
  // Q stays at offset 0: the loop's Q reads then fit the LDS instructions' immediate offsets.
  constexpr int kOOff = kOwn ? (kQBytes + 15) / 16 * 16 : 0;
  constexpr int kLdsBytes = kOwn ? kOOff + kOBytes : (kQBytes > kOBytes ? kQBytes : kOBytes);
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];
  unsigned char* const qsh = lds;
  __shared__ float sm_m[kWaves][kRows];
  __shared__ float sm_l[kWaves][kRows];
  __shared__ float sm_M[kRows];
  __shared__ float sm_L[kRows];
  __shared__ int sm_plan[4];
  float* osh = reinterpret_cast<float*>(lds + kOOff);
  const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // The block table is read-only here: reading it through the constant address space lets
  // the wave-uniform page lookups be scalar loads, which do not wait behind (or drain) the
  // wave's outstanding K/V vector loads.
  typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
  const int64_t bt_last = bt_stride - 1;
  // The pages of the wave's first tile of piece sidx of sequence b, looked up before L is
  // known: they are used only if that tile is full, i.e. all its keys are < L, where no
  // clamp to L - 1 applies (the index is kept inside the table row regardless).
  auto first_pages = [&](int b, int sidx, int32_t& p0, int32_t& p1) {
    const const_i32_ptr tb = (const_i32_ptr)(bt_p + static_cast<int64_t>(b) * bt_stride);
    const int kb = sidx * split + wave * kTileKeys;
    p0 = tb[min<int64_t>(kb >> bs_shift, bt_last)];
    p1 = tb[min<int64_t>((kb + 16) >> bs_shift, bt_last)];
  };

  // One piece: keys [sidx * split, min(L, (sidx + 1) * split)) of (sequence b, KV head hkv)
  // with query rows [q0, q0 + n); L = min(seq_lens[b], max_seqlen_k); pg0 / pg1 the pages of
  // the wave's first tile (first_pages).
  auto run_piece = [&](const int b, const int hkv, const int sidx, const int q0, const int n,
                       const int L, const int32_t pg0, const int32_t pg1) {
  const const_i32_ptr table = (const_i32_ptr)(bt_p + static_cast<int64_t>(b) * bt_stride);
  const int k_begin = sidx * split;
  const int64_t first_pg0 = clamp_page(pg0, a.num_blocks);
  const int64_t first_pg1 = clamp_page(pg1, a.num_blocks);
  if (n <= 0) return;
  const int nsplit = L > 0 ? (L + split - 1) / split : 1;
  if (sidx >= nsplit) return;
  const int R = min(min(a.G * n, kRows), a.rmax);
  const int k_end = min(L, k_begin + split);

  const int bs_mask = (1 << bs_shift) - 1;

  // ---- Q rows (into LDS by stage_q, once the first tile's loads are issued), causal limits ----
  // Row r of the block is query head hkv*G + r/n at query row j = r % n; rows >= R are 0.
  constexpr int kQCh = D / 8;  // 16-byte chunks per row
  constexpr int kQIter = (kRows * kQCh + kBlock - 1) / kBlock;
  u32x4_t qreg[kQIter];
  constexpr bool fused = FUSED != 0;
#pragma unroll
  for (int it = 0; it < kQIter; ++it) {
    const int idx = it * kBlock + tid;
    const int r = idx / kQCh, c = idx % kQCh;
    qreg[it] = u32x4_t{0, 0, 0, 0};
    if (r < R && !fused) {
      const int hl = r / n, j = r - hl * n;
      qreg[it] = *reinterpret_cast<const u32x4_t*>(a.q + static_cast<int64_t>(q0 + j) * a.q_ts +
                                                   static_cast<int64_t>(hkv * a.G + hl) * a.q_hs + c * 8);
    }
  }
  // Fused epilogue (engine/model.py:238-243 for this block's rows): every G-lane group
  // (G = D/8) takes one vector -- a q head of a row (RoPE, into the LDS row stage_q would
  // fill) or a row's k and v of this KV head (RoPE on k, then the cache write of
  // reshape_and_cache_flash, INT8 quantised as coopt_kv_write does).  stage_q's barrier
  // orders these cache writes before any of the block's loads of the new keys; a wave's first
  // tile is loaded before that barrier only if it holds none of them.
  auto fused_epilogue = [&]() {
    constexpr int GL = D / 8;
    const int nq = a.G * n, nvec = nq + n;
    const int Hq = a.G * a.Hkv;
    const int width = (Hq + 2 * a.Hkv) * D;
    const int64_t num_slots = a.num_blocks << bs_shift;
    for (int base = 0; base < nvec * GL; base += kBlock) {  // uniform trip count
      const int lid = base + tid;
      const int vi = lid / GL, c = lid % GL;
      if (vi >= nvec) continue;  // whole groups: nvec * GL is a multiple of GL
      const bool is_kv = vi >= nq;
      const int j = is_kv ? vi - nq : vi % n;
      const int hl = is_kv ? 0 : vi / n;
      const int t = q0 + j;
      const int head = is_kv ? Hq + hkv : hkv * a.G + hl;
      // The RoPE rows of the row's key position L - n + j, which is its position in every
      // step; loaded with the partials, and again below only if positions[t] says otherwise
      const int64_t p_key = L - n + j;
      RopeTab tab = rope_tab<GL>(a.cos, a.sin, a.tab_stride, p_key, a.max_pos, c);
      const int64_t p = a.pos[t];
      const int64_t slot_t = a.slots[t];
      const int64_t slot = is_kv ? slot_t : -1;
      const int64_t col = static_cast<int64_t>(head) * D + c * 8;
      // q lanes point their (unused) v loads at their own x chunk: every load is issued
      // unconditionally, and before any value is used
      const int64_t vcol = is_kv ? static_cast<int64_t>(Hq + a.Hkv + hkv) * D + c * 8 : col;
      uint4 xr, vr;
      if constexpr (FUSED == 2) {
        // the same order of adds as the reduction of coopt_linear's partials
        const float* pr = static_cast<const float*>(a.qkv_src) + static_cast<int64_t>(t) * width;
        Partials4<kQkvMaxSlices> xlo, xhi, vlo, vhi;
        xlo.load(pr + col, a.qkv_ks, a.qkv_stride);
        xhi.load(pr + col + 4, a.qkv_ks, a.qkv_stride);
        vlo.load(pr + vcol, a.qkv_ks, a.qkv_stride);
        vhi.load(pr + vcol + 4, a.qkv_ks, a.qkv_stride);
        auto pack8 = [&](const Partials4<kQkvMaxSlices>& lo, const Partials4<kQkvMaxSlices>& hi) {
          const float4 l = lo.sum(a.qkv_ks), h = hi.sum(a.qkv_ks);
          return make_uint4(pack2_bf16(l.x, l.y), pack2_bf16(l.z, l.w), pack2_bf16(h.x, h.y),
                            pack2_bf16(h.z, h.w));
        };
        xr = pack8(xlo, xhi);
        vr = pack8(vlo, vhi);
      } else {
        const uint16_t* rr = static_cast<const uint16_t*>(a.qkv_src) + static_cast<int64_t>(t) * a.qkv_stride;
        xr = *reinterpret_cast<const uint4*>(rr + col);
        vr = *reinterpret_cast<const uint4*>(rr + vcol);
      }
      if (clamp_pos(p, a.max_pos) != clamp_pos(p_key, a.max_pos))
        tab = rope_tab<GL>(a.cos, a.sin, a.tab_stride, p, a.max_pos, c);
      const uint4 yr = rope_chunk<GL>(xr, tab, c);
      if (!is_kv) {
        // rows past R (a sequence with more rows than max_seqlen_q) are not attended; their
        // store would land past the Q rows
        const int r = hl * n + j;
        if (r < R) *reinterpret_cast<uint4*>(qsh + r * kQPitch + c * 16) = yr;
      } else if (slot >= 0 && slot < num_slots) {  // padding rows write nothing
        const int64_t blk = slot >> bs_shift;
        const int64_t off = slot & bs_mask;
        store_kv_chunk<GL, INT8>(yr, vr, const_cast<void*>(a.kc), const_cast<void*>(a.vc),
                                 blk * a.c_bs + off * a.c_ts + hkv * a.c_hs + c * 8,
                                 const_cast<uint16_t*>(a.ks), const_cast<uint16_t*>(a.vs),
                                 blk * a.s_bs + off * a.s_ts + hkv * a.s_hs, c);
      }
    }
    // Q rows past R are zero, as stage_q leaves them
    for (int idx = tid; idx < (kRows - R) * kQCh; idx += kBlock) {
      const int r = R + idx / kQCh, c = idx % kQCh;
      *reinterpret_cast<u32x4_t*>(qsh + r * kQPitch + c * 16) = u32x4_t{0, 0, 0, 0};
    }
  };
  // Run here, before the attention's own state is set up: its scalars (kernel-argument
  // fields) are dead again by the time the loop's page bases and offsets are live.  (Run
  // after the first tile's loads are issued, to overlap them, it made the compiler move
  // ~35 scalars into vector-register lanes and measured slower.)
  if constexpr (FUSED) fused_epilogue();
  auto stage_q = [&]() {
    if (!fused) {
#pragma unroll
      for (int it = 0; it < kQIter; ++it) {
        const int idx = it * kBlock + tid;
        const int r = idx / kQCh, c = idx % kQCh;
        if (r < kRows) *reinterpret_cast<u32x4_t*>(qsh + r * kQPitch + c * 16) = qreg[it];
      }
    }
    __syncthreads();
  };
  const float score_scale = a.scale_log2;
  int lim[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 16 + l16;
    lim[rt] = r < R ? L - n + (r % n) : -1;  // bottom-right aligned causal mask
  }
  // the lane's Q operand of (rt, ks): row rt*16 + l16, the 8 elements from d_of(ks) (the
  // contraction map of the K loads)
  const unsigned char* qlds = qsh + l16 * kQPitch;
  auto q_byte = [&](int ks) {
    return INT8 ? 2 * (64 * (ks >> 1) + 16 * grp + 8 * (ks & 1)) : 2 * (32 * ks + 8 * grp);
  };

  f32x4_t o[RT][kDt];
  float m_run[RT], l_run[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt) o[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // INT8: the wave's V-scale reference exponent e_v (wave-uniform).  The PV operand is
  // fp16(p * s_v * 2^-e_v); o and l are kept relative to 2^(m_run + e_v), so e_v enters the
  // exponent of p and the row maxima the merge sees, and cancels in o / l.
  int e_v = 0;
  bool ev_set = false;

  const int ntiles = (k_end - k_begin + kTileKeys - 1) / kTileKeys;
  const unsigned char* kbase = static_cast<const unsigned char*>(a.kc);
  const unsigned char* vbase = static_cast<const unsigned char*>(a.vc);
  const int64_t head_off = static_cast<int64_t>(hkv) * a.c_hs;
  const int64_t shead_off = static_cast<int64_t>(hkv) * a.s_hs;
  const int min_lim = L - n;  // causal limit of the first query row

  // `wave` is uniform, so tile bookkeeping and page lookups are scalar.  A 32-key tile starts
  // on a multiple of 32 and block_size >= 16, so its keys lie in at most two pages: the page
  // of key kb (sub-tile 0) and of key kb + 16 (sub-tile 1); keys past the end are clamped to
  // L - 1, which stays in the page of its 16-key sub-tile.
  auto page_of = [&](int key) {
    return clamp_page(table[min(key, L - 1) >> bs_shift], a.num_blocks);
  };

  // Issue every load of tile `t` (pages pg0/pg1).  Page bases are wave-uniform (scalar);
  // lanes add 32-bit byte offsets.  Full tiles (every key < L) use offsets fixed for the
  // whole loop; the last, partial tile clamps each key to L - 1, so no row past the
  // sequence is read.
  const int c_ts = static_cast<int>(a.c_ts), s_ts = static_cast<int>(a.s_ts);
  const uint32_t k_lane = kElt * l16 * c_ts + 16 * grp;
  uint32_t v_lane[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v_lane[i] = kElt * ((grp * 4 + i) * c_ts + l16 * kDt);
  // The empty asm keeps each offset a 32-bit register at its use, so the loads take the
  // scalar-base + 32-bit-offset form instead of a per-lane 64-bit address.
  auto issue = [&](Raw& raw, int kt, const unsigned char* kp, const unsigned char* vp,
                   uint32_t ko, const uint32_t (&vo)[4]) {
#pragma unroll
    for (int c = 0; c < Raw::kKVec; ++c) {
      uint32_t off = ko + 64u * c;
      asm volatile("" : "+v"(off));
      raw.k[kt][c] = *reinterpret_cast<const u32x4_t*>(kp + off);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t off = vo[i];
      asm volatile("" : "+v"(off));
      load_words<Raw::kVWords>(vp + off, raw.v[kt * 4 + i]);
    }
  };
  // a full tile: every key < L
  // INT8: the scales are issued first, so the V-scale check of a loaded tile (vcheck) waits
  // only for them and leaves the tile's K/V loads in flight.
  auto load_full = [&](Raw& raw, int t, int64_t pg0, int64_t pg1) {
    const int kb = k_begin + t * kTileKeys;
    if constexpr (INT8) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int64_t pg = kt ? pg1 : pg0;
        const int tok0 = (kb + kt * 16) & bs_mask;
        const uint16_t* ksp = a.ks + pg * a.s_bs + shead_off;
        const uint16_t* vsp = a.vs + pg * a.s_bs + shead_off;
        if constexpr (SC) {
          uint32_t ko2 = l16 * 2, vo2 = grp * 8;
          asm volatile("" : "+v"(ko2), "+v"(vo2));
          raw.ks[kt] = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const unsigned char*>(ksp + tok0) + ko2);
          raw.vs[kt] = *reinterpret_cast<const u32x2_t*>(reinterpret_cast<const unsigned char*>(vsp + tok0) + vo2);
        } else {
          raw.ks[kt] = ksp[(tok0 + l16) * s_ts];
          uint32_t vh[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) vh[i] = vsp[(tok0 + grp * 4 + i) * s_ts];
          raw.vs[kt] = u32x2_t{vh[0] | (vh[1] << 16), vh[2] | (vh[3] << 16)};
        }
      }
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int64_t pg = kt ? pg1 : pg0;
      const int tok0 = (kb + kt * 16) & bs_mask;
      const int64_t r = pg * a.c_bs + head_off + static_cast<int64_t>(tok0) * c_ts;
      issue(raw, kt, kbase + kElt * r, vbase + kElt * r, k_lane, v_lane);
    }
  };
  // the split's last tile when it ends inside a tile: keys clamped to L - 1
  auto load_partial = [&](Raw& raw, int t, int64_t pg0, int64_t pg1) {
    const int kb = k_begin + t * kTileKeys;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int64_t pg = kt ? pg1 : pg0;
      const int sub = kb + kt * 16;
      const int64_t row0 = pg * a.c_bs + head_off;
      const int ktk = min(sub + l16, L - 1) & bs_mask;
      const uint32_t ko = kElt * ktk * c_ts + 16 * grp;
      uint32_t vo[4], tk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        tk[i] = min(sub + grp * 4 + i, L - 1) & bs_mask;
        vo[i] = kElt * (tk[i] * c_ts + l16 * kDt);
      }
      issue(raw, kt, kbase + kElt * row0, vbase + kElt * row0, ko, vo);
      if constexpr (INT8) {
        const uint16_t* ksp = a.ks + pg * a.s_bs + shead_off;
        const uint16_t* vsp = a.vs + pg * a.s_bs + shead_off;
        raw.ks[kt] = ksp[ktk * s_ts];
        uint32_t vh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) vh[i] = vsp[tk[i] * s_ts];
        raw.vs[kt] = u32x2_t{vh[0] | (vh[1] << 16), vh[2] | (vh[3] << 16)};
      }
    }
  };

  // INT8: keep fp16(p * s_v * 2^-e_v) in range.  p <= 2^kSlack = 2^8, so every V scale must
  // stay at or below 2^(e_v + 7) (products <= 2^15 < 65504).  The first positive scale, or
  // one above that bound, moves e_v so that the tile's largest scale lands in [2^6, 2^7),
  // and o and l are rescaled by the change (one uniform branch, taken O(log range) times
  // per wave).  Scales are non-negative fp16, so their bit patterns order them; non-finite
  // patterns count as the largest finite scale.  Run on a tile before it is computed, at the
  // end of the previous tile's compute, where that tile's registers are free.
  auto vcheck = [&](const Raw& raw) {
    if constexpr (INT8) {
      const uint32_t wv = max_u16x2(max_u16x2(raw.vs[0][0], raw.vs[0][1]),
                                    max_u16x2(raw.vs[1][0], raw.vs[1][1]));
      const uint32_t smax = min(max(wv & 0xffffu, wv >> 16), 0x7bffu);
      const uint32_t thr = !ev_set ? 0u
                           : (e_v + 7 >= 16 ? 0x7c00u : static_cast<uint32_t>(e_v + 7 + 15) << 10);
      if (__builtin_amdgcn_ballot_w64(smax > thr)) {
        uint32_t wm = smax;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1)
          wm = max(wm, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wm), off, 64)));
        // fp16 exponent of the largest scale (subnormals count as 2^-15), minus 6
        const int e_new = __builtin_amdgcn_readfirstlane(static_cast<int>(wm >> 10) - 21);
        const float f = exp2_fast(static_cast<float>(e_v - e_new));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          l_run[rt] *= f;
#pragma unroll
          for (int dt = 0; dt < kDt; ++dt) o[rt][dt] *= f;
        }
        e_v = e_new;
        ev_set = true;
      }
    }
  };

  auto compute_tile = [&](const Raw& raw, int t) {
    const int kb = k_begin + t * kTileKeys;
    // every key of the tile inside the split and visible to every row: no masking
    const bool open = kb + kTileKeys <= k_end && kb + kTileKeys - 1 <= min_lim;
    auto scale_of = [&](const u32x2_t& w, int i) {
      return f16_to_f32(static_cast<uint16_t>(w[i >> 1] >> (16 * (i & 1))));
    };
    constexpr uint32_t k64 = 0x64646464u;  // fp16 exponent bytes of 1024

    // ---- V^T operands.  They do not depend on the scores: up to 32 rows they are built
    // first, so their VALU work is scheduled alongside the score MFMAs in one basic block;
    // at 48 rows and more they are built after the softmax, which keeps them out of the
    // score phase's registers ----
    u32x4_t va[kDt];
    auto build_va = [&]() {
      uint32_t vx[8][Raw::kVWords];
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int w = 0; w < Raw::kVWords; ++w) vx[j][w] = INT8 ? (raw.v[j][w] ^ 0x80808080u) : raw.v[j][w];
      if constexpr (INT8) {
        // exact fp16 codes; the V scales go into P (below).  Two byte selects interleave
        // keys j0, j1 over four d's, two more place each pair under the 0x64 exponent bytes.
#pragma unroll
        for (int w = 0; w < Raw::kVWords; ++w)
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int j0 = 2 * e2, j1 = 2 * e2 + 1;  // keys of k-elements 2*e2, 2*e2+1
            const uint32_t lo = __builtin_amdgcn_perm(vx[j1][w], vx[j0][w], 0x05010400u);
            const uint32_t hi = __builtin_amdgcn_perm(vx[j1][w], vx[j0][w], 0x07030602u);
            va[4 * w + 0][e2] = codes_f16x2(__builtin_amdgcn_perm(k64, lo, 0x04010400u));
            va[4 * w + 1][e2] = codes_f16x2(__builtin_amdgcn_perm(k64, lo, 0x04030402u));
            va[4 * w + 2][e2] = codes_f16x2(__builtin_amdgcn_perm(k64, hi, 0x04010400u));
            va[4 * w + 3][e2] = codes_f16x2(__builtin_amdgcn_perm(k64, hi, 0x04030402u));
          }
      } else {
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int j0 = 2 * e2, j1 = 2 * e2 + 1;  // keys of k-elements 2*e2, 2*e2+1
            const int w = dt >> 1;
            va[dt][e2] = __builtin_amdgcn_perm(vx[j1][w], vx[j0][w], (dt & 1) ? 0x07060302u : 0x05040100u);
          }
      }
    };
    constexpr bool kVFirst = RT <= 2;
    if constexpr (kVFirst) build_va();

    // ---- scores: S^T = K . Q^T, K operands built per k-step ----
    f32x4_t acc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt][0] = acc[rt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) {
      u32x4_t qop[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        qop[rt] = *reinterpret_cast<const u32x4_t*>(qlds + rt * 16 * kQPitch + q_byte(ks));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        u32x4_t kop;
        if constexpr (INT8) {
          // the lane's key l16 of sub-tile kt: codes 8*(ks%2) .. +8 of its load ks/2
          const u32x4_t& c4 = raw.k[kt][ks >> 1];
          const float sk = f16_to_f32(static_cast<uint16_t>(raw.ks[kt]));
          const float skb = -1152.0f * sk;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t ux = c4[(ks & 1) * 2 + h] ^ 0x80808080u;
            kop[2 * h] = dequant_pair(__builtin_amdgcn_perm(k64, ux, 0x04010400u), sk, skb);
            kop[2 * h + 1] = dequant_pair(__builtin_amdgcn_perm(k64, ux, 0x04030402u), sk, skb);
          }
        } else {
          kop = raw.k[kt][ks];
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][kt] = mfma_bf16(kop, qop[rt], acc[rt][kt]);
      }
    }

    // ---- online softmax (log2 domain) ----
    // m_run is a per-row reference max that is raised only when a score exceeds it by more
    // than kSlack: exponents are then at most 2^kSlack (exact range for bf16 P and the fp32
    // sums), and the accumulators are rescaled only on those rare raises (one branch per
    // tile, taken by the whole wave).
    constexpr float kSlack = 8.0f;
    float sv[RT][2][4];  // raw scores (the scale is applied in the exponent); masked -inf
    if (open) {  // one uniform branch for the whole tile
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[rt][kt][i] = acc[rt][kt][i];
    } else {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + kt * 16 + grp * 4 + i;
            sv[rt][kt][i] = (key > lim[rt] || key >= k_end) ? -INFINITY : acc[rt][kt][i];
          }
    }
    float m_tile[RT];
    bool raise_any = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float tmax = fmaxf(fmaxf(fmaxf(sv[rt][0][0], sv[rt][0][1]), fmaxf(sv[rt][0][2], sv[rt][0][3])),
                         fmaxf(fmaxf(sv[rt][1][0], sv[rt][1][1]), fmaxf(sv[rt][1][2], sv[rt][1][3])));
      tmax = max_xor32(max_xor16(tmax));
      m_tile[rt] = tmax * score_scale;
      raise_any |= m_tile[rt] > m_run[rt] + kSlack;
    }
    if (__builtin_amdgcn_ballot_w64(raise_any)) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const bool raise = m_tile[rt] > m_run[rt] + kSlack;
        const float m_new = raise ? m_tile[rt] : m_run[rt];
        const float alpha = raise ? exp2_fast(m_run[rt] - m_new) : 1.0f;  // 0 when raised from -inf
        l_run[rt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt) o[rt][dt] *= alpha;
        m_run[rt] = m_new;
      }
    }
    uint32_t pb[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float m_use = (m_run[rt] == -INFINITY ? 0.0f : m_run[rt]) +
                          (INT8 ? static_cast<float>(e_v) : 0.0f);
      float p[2][4], psum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[kt][i] = exp2_fast(fmaf(sv[rt][kt][i], score_scale, -m_use));
          psum += p[kt][i];
        }
      l_run[rt] += psum;
      if constexpr (INT8) {
        // P' = p * s_v of the lane's key j = 4 kt + i, in fp16 next to the fp16 codes
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) p[kt][i] *= scale_of(raw.vs[kt], i);
        pb[rt][0] = pack_f16x2(p[0][0], p[0][1]);
        pb[rt][1] = pack_f16x2(p[0][2], p[0][3]);
        pb[rt][2] = pack_f16x2(p[1][0], p[1][1]);
        pb[rt][3] = pack_f16x2(p[1][2], p[1][3]);
      } else {
        pb[rt][0] = pack_bf16x2(p[0][0], p[0][1]);
        pb[rt][1] = pack_bf16x2(p[0][2], p[0][3]);
        pb[rt][2] = pack_bf16x2(p[1][0], p[1][1]);
        pb[rt][3] = pack_bf16x2(p[1][2], p[1][3]);
      }
    }

    if constexpr (!kVFirst) build_va();

    // ---- O^T += V^T . P^T ----
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const u32x4_t pbv = {pb[rt][0], pb[rt][1], pb[rt][2], pb[rt][3]};
        o[rt][dt] = INT8 ? mfma_f16(va[dt], pbv, o[rt][dt]) : mfma_bf16(va[dt], pbv, o[rt][dt]);
      }
  };

  // ---- the wave's tiles: double-buffered (the next tile's loads in flight while the current
  // one is computed) or, for large row counts, one at a time; then the partial tile ----
  // Wave w takes tiles w, w + kWaves, w + 2 kWaves, ... (a fixed assignment keeps the result
  // bit-reproducible: each wave's sum covers the same keys on every call); the wave whose
  // sequence reaches nfull also takes the split's partial tile.
  const int nfull = (k_end - k_begin) / kTileKeys;
  auto pages = [&](int t, int64_t& p0, int64_t& p1) {
    const int kb = k_begin + t * kTileKeys;
    p0 = page_of(kb);
    p1 = page_of(kb + 16);
  };
  bool own_partial = wave == nfull;
  int next_t = wave + kWaves;
  auto grab = [&]() {
    const int v = next_t;
    next_t += kWaves;
    own_partial |= v == nfull;
    return v;
  };
  if constexpr (DB) {
    // Loads inside the loop are unconditional (an index past the last full tile repeats it,
    // already cached, and is never computed), so each compute waits only for its own
    // buffer's loads and the other buffer's stay in flight.
    Raw bufA, bufB;
    const int tlast = nfull - 1;
    int tA = wave;
    int64_t nx0 = 0, nx1 = 0;  // pages of the wave's next tile to load
    // fused: a first tile holding keys this launch writes ([L - n, L)) loads after the barrier
    const bool defer = fused && k_begin + (tA + 1) * kTileKeys > L - n;
    if (tA < nfull && !defer) load_full(bufA, tA, first_pg0, first_pg1);
    stage_q();  // the Q loads complete while the first tile's are in flight
    if (tA < nfull && defer) load_full(bufA, tA, first_pg0, first_pg1);
    if (tA < nfull) {
      vcheck(bufA);
      int tB = grab();
      pages(min(tB, tlast), nx0, nx1);
      for (;;) {
        load_full(bufB, min(tB, tlast), nx0, nx1);
        const int tA2 = tB < nfull ? grab() : nfull;
        pages(min(tA2, tlast), nx0, nx1);
        compute_tile(bufA, tA);
        vcheck(bufB);
        if (tB >= nfull) break;
        load_full(bufA, min(tA2, tlast), nx0, nx1);
        const int tB2 = tA2 < nfull ? grab() : nfull;
        pages(min(tB2, tlast), nx0, nx1);
        compute_tile(bufB, tB);
        vcheck(bufA);
        if (tA2 >= nfull) break;
        tA = tA2;
        tB = tB2;
      }
    }
  } else {
    Raw buf;
    int64_t nx0 = 0, nx1 = 0;
    int t = wave;
    if (t < nfull) {
      nx0 = first_pg0;
      nx1 = first_pg1;
    }
    stage_q();
    while (t < nfull) {
      load_full(buf, t, nx0, nx1);
      const int tn = grab();
      if (tn < nfull) pages(tn, nx0, nx1);
      vcheck(buf);
      compute_tile(buf, t);
      t = tn;
    }
  }
  if (nfull < ntiles && own_partial) {
    Raw buf;
    int64_t p0, p1;
    pages(nfull, p0, p1);
    load_partial(buf, nfull, p0, p1);
    vcheck(buf);
    compute_tile(buf, nfull);
  }
  // ---- merge the waves ----
  // the wave's o and l are relative to 2^(m_run + e_v) (e_v = 0 for bf16 KV)
  const float ev_f = INT8 ? static_cast<float>(e_v) : 0.0f;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] += ev_f;
    l_run[rt] = add_xor32(add_xor16(l_run[rt]));
  }
  // lane's accumulators: row rt*16 + l16, d = (4g + i) * kDt + dt -- kDt contiguous floats
  // for each (rt, i); stored into `region` (add: onto what an earlier wave stored there)
  auto store_acc = [&](float* region, bool add) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int r = rt * 16 + l16;
      if (rt * 16 >= R) break;  // row tiles of padding only (uniform)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* dst = region + r * kOPitch + (grp * 4 + i) * kDt;
#pragma unroll
        for (int d4 = 0; d4 < kDt / 4; ++d4) {
          const f32x4_t x = {o[rt][d4 * 4 + 0][i], o[rt][d4 * 4 + 1][i], o[rt][d4 * 4 + 2][i],
                             o[rt][d4 * 4 + 3][i]};
          f32x4_t* dp = reinterpret_cast<f32x4_t*>(dst + 4 * d4);
          if (!add) *dp = x;
          else *dp = *dp + x;
        }
      }
    }
  };
  if constexpr (kOwn) {
    // no wait for the other waves: the region and the (m, l) slots are this wave's alone
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (grp == 0) {
        sm_m[wave][rt * 16 + l16] = m_run[rt];
        sm_l[wave][rt * 16 + l16] = l_run[rt];
      }
    }
    store_acc(osh + wave * kRegionFloats, false);
    __syncthreads();
  } else {
    __syncthreads();  // Q in LDS is dead; the merge below reuses the space
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
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
      for (int dt = 0; dt < kDt; ++dt) o[rt][dt] *= f;
      if (wave == 0 && grp == 0) {
        sm_M[r] = M;
        sm_L[r] = Lsum;
      }
    }
    // wave w stores into region w % kRegions in round w / kRegions (later rounds add); the
    // output pass sums the regions in order
#pragma unroll
    for (int round = 0; round < kWaves / kRegions; ++round) {
      if (wave / kRegions == round) store_acc(osh + (wave % kRegions) * kRegionFloats, round > 0);
      __syncthreads();
    }
  }
  // row r, elements [8c, 8c + 8) of the merged (unnormalised) output, relative to 2^M, and
  // the row's (M, L)
  auto merged8 = [&](int r, int c, f32x4_t& lo, f32x4_t& hi, float& M, float& Lsum) {
    const float* src = osh + r * kOPitch + c * 8;
    if constexpr (kOwn) {
      M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][r]);
      Lsum = 0.0f;
      lo = f32x4_t{0.f, 0.f, 0.f, 0.f};
      hi = lo;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = sm_m[w][r];
        const float f = mw > -INFINITY ? exp2_fast(mw - M) : 0.0f;
        Lsum += sm_l[w][r] * f;
        lo += *reinterpret_cast<const f32x4_t*>(src + w * kRegionFloats) * f;
        hi += *reinterpret_cast<const f32x4_t*>(src + w * kRegionFloats + 4) * f;
      }
    } else {
      M = sm_M[r];
      Lsum = sm_L[r];
      lo = *reinterpret_cast<const f32x4_t*>(src);
      hi = *reinterpret_cast<const f32x4_t*>(src + 4);
#pragma unroll
      for (int g = 1; g < kRegions; ++g) {
        lo += *reinterpret_cast<const f32x4_t*>(src + g * kRegionFloats);
        hi += *reinterpret_cast<const f32x4_t*>(src + g * kRegionFloats + 4);
      }
    }
  };

  constexpr int kCh = D / 8;  // 8-element chunks per row
  if (nsplit == 1) {
    for (int idx = tid; idx < R * kCh; idx += kBlock) {
      const int r = idx / kCh, c = idx % kCh;
      f32x4_t lo, hi;
      float Mr, Lr;
      merged8(r, c, lo, hi, Mr, Lr);
      const float inv = Lr > 0.0f ? 1.0f / Lr : 0.0f;
      u32x4_t v;
      v[0] = pack_bf16x2(lo[0] * inv, lo[1] * inv);
      v[1] = pack_bf16x2(lo[2] * inv, lo[3] * inv);
      v[2] = pack_bf16x2(hi[0] * inv, hi[1] * inv);
      v[3] = pack_bf16x2(hi[2] * inv, hi[3] * inv);
      const int hl = r / n, j = r - hl * n;
      uint16_t* dst = a.out + static_cast<int64_t>(q0 + j) * a.o_ts +
                      static_cast<int64_t>(hkv * a.G + hl) * a.o_hs + c * 8;
      *reinterpret_cast<u32x4_t*>(dst) = v;
    }
    return;
  }

  // ---- several splits: publish this split's partial; merge_kernel combines them ----
  const int64_t pbase = ((static_cast<int64_t>(b) * a.Hkv + hkv) * a.max_splits + sidx) * a.rmax;
  for (int idx = tid; idx < R * kCh; idx += kBlock) {
    const int r = idx / kCh, c = idx % kCh;
    f32x4_t lo, hi;
    float Mr, Lr;
    merged8(r, c, lo, hi, Mr, Lr);
    float* dst = a.part_o + (pbase + r) * D + c * 8;
    reinterpret_cast<f32x4_t*>(dst)[0] = lo;
    reinterpret_cast<f32x4_t*>(dst)[1] = hi;
    if (c == 0) a.part_ml[pbase + r] = make_float2(Mr, Lr);
  }
  };  // run_piece

  // Clamps keep a malformed call (seq_len > max_seqlen_k, q_len > max_seqlen_q, block ids
  // outside the pool) inside its buffers: such calls give wrong rows, never stray accesses.
  int b, hkv, sidx, q0, n, L;
  int32_t pg0, pg1;
  if (mode == 1) {  // a.plan
    if (wave == 0) plan_item(a, lane, sm_plan);
    __syncthreads();
    b = __builtin_amdgcn_readfirstlane(sm_plan[0]);
    q0 = __builtin_amdgcn_readfirstlane(sm_plan[1]);
    n = __builtin_amdgcn_readfirstlane(sm_plan[2]);
    L = __builtin_amdgcn_readfirstlane(sm_plan[3]);
    hkv = static_cast<int>(blockIdx.x) % a.Hkv;
    sidx = 0;
    first_pages(b, sidx, pg0, pg1);
  } else if (mode == 2) {  // a.nwin > 0
    const int x = static_cast<int>(blockIdx.x);
    hkv = x % a.Hkv;
    const int rest = x / a.Hkv;
    b = rest / a.nwin;
    const int w = rest - b * a.nwin;
    sidx = 0;
    const const_i32_ptr cuc = (const_i32_ptr)cu_p;
    const const_i32_ptr slc = (const_i32_ptr)sl_p;
    const int c0 = cuc[b], c1 = cuc[b + 1], sl = slc[b];
    first_pages(b, sidx, pg0, pg1);
    const int nall = c1 - c0, j0 = w * a.qwin;
    n = min(max(nall - j0, 0), a.qwin);
    q0 = c0 + j0;
    // keys [0, L) end where the window's last row's causal limit does
    L = min(sl, a.max_seqlen_k) - (nall - j0 - n);
  } else {
    b = blockIdx.z;
    hkv = blockIdx.y;
    sidx = blockIdx.x;
    // every scalar the block's first loads depend on, in one round: the row range, the key
    // count and the first tile's pages, and the kernel-argument lines the Q / K / V (or
    // epilogue) addressing reads.  The empty asm keeps these loads from being spread over the
    // code that uses them, each behind a wait of its own.
    const const_i32_ptr cuc = (const_i32_ptr)cu_p;
    const const_i32_ptr slc = (const_i32_ptr)sl_p;
    const int c0 = cuc[b], c1 = cuc[b + 1], sl = slc[b];
    first_pages(b, sidx, pg0, pg1);
    const void* line4 = FUSED != 0 ? static_cast<const void*>(a.slots) : static_cast<const void*>(a.q);
    asm volatile("" ::"s"(c0), "s"(c1), "s"(sl), "s"(pg0), "s"(pg1), "s"(a.kc), "s"(line4));
    q0 = c0;
    n = c1 - c0;
    L = min(sl, a.max_seqlen_k);
  }
  run_piece(b, hkv, sidx, q0, n, L, pg0, pg1);
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
  const int64_t first = (static_cast<int64_t>(b) * a.Hkv + hkv) * a.max_splits;
  auto slot = [&](int s) { return (first + s) * a.rmax; };
  for (int idx = threadIdx.x; idx < R * kCh; idx += kThreads) {
    const int r = idx / kCh, c = idx % kCh;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.part_ml[slot(s) + r].x);
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float Lsum = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
      const float2 ml = a.part_ml[slot(s) + r];
      if (!(ml.x > -INFINITY)) continue;
      const float w = exp2_fast(ml.x - M);
      Lsum += ml.y * w;
      const f32x4_t* src = reinterpret_cast<const f32x4_t*>(a.part_o + (slot(s) + r) * D + c * 8);
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
// reading seq_lens.  Aims at one block per CU (8-wave blocks) or two (4-wave blocks) for the
// longest context, in whole rounds of 32-key tiles over the block's waves; a sequence longer
// than one split is split, so shorter ones run whole.
int target_blocks(int waves) { return waves == 8 ? 256 : 512; }

int choose_split(int B, int Hkv, int max_seqlen_k, int waves) {
  const int64_t items = static_cast<int64_t>(B) * Hkv;
  const int64_t target = target_blocks(waves);
  const int64_t gran = 32 * waves;
  int64_t per = (static_cast<int64_t>(max_seqlen_k) * items + target - 1) / target;
  per = ((per + gran - 1) / gran) * gran;
  if (per < 2 * gran) per = 2 * gran;
  if (per > 65536) per = 65536;
  return static_cast<int>(per);
}

// How one call is laid out: `split`-key pieces, max_splits per (sequence, KV head).  plan:
// more (sequence, KV head) items than one round of blocks holds, none split, B <= kPlanSeqs --
// a 1-D grid of B * Hkv blocks that order the items themselves (plan_item); otherwise the
// grid (max_splits, Hkv, B) in order, where one round holds every item and order is moot.
// Windowed launches (query windows, see AttnArgs): more than kMaxRows rows per KV head.
struct AttnShape {
  bool plan;
  int split, max_splits;
  int rmax;        // rows per (item, KV head): G * max_seqlen_q, or G * qwin when windowed
  int qwin, nwin;  // windowed: rows per window and windows per sequence (else 0, 0)
};

constexpr int kMaxRows = 64;

AttnShape attn_shape(int B, int G, int Hkv, int max_seqlen_q, int max_seqlen_k) {
  AttnShape s{};
  if (G * static_cast<int64_t>(max_seqlen_q) > kMaxRows) {
    // prefill-sized rows (a chunk of a mixed batch, a long catch-up): windows of kMaxRows / G
    // rows, each one unsplit block -- correct at any length, not tuned for throughput
    s.qwin = kMaxRows / G;
    s.nwin = (max_seqlen_q + s.qwin - 1) / s.qwin;
    s.rmax = G * s.qwin;
    const int gran = 32 * waves_for((s.rmax + 15) / 16);
    s.split = static_cast<int>((static_cast<int64_t>(max_seqlen_k) + gran - 1) / gran * gran);
    s.max_splits = 1;
    s.plan = false;
    return s;
  }
  s.rmax = G * max_seqlen_q;
  const int waves = waves_for((s.rmax + 15) / 16);
  s.split = choose_split(B, Hkv, max_seqlen_k, waves);
  s.max_splits = (max_seqlen_k + s.split - 1) / s.split;
  s.plan = B <= kPlanSeqs && static_cast<int64_t>(B) * Hkv > target_blocks(waves) &&
           s.max_splits == 1;
  return s;
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

// Shapes the fused epilogue is instantiated for: up to 32 rows (a speculative step's verify
// and draft shapes), except bf16 at head dim 128 with 32 rows, which would spill registers.
constexpr int kFusedMaxRT = 2;
constexpr bool fused_ok(int D, bool int8, int RT) {
  return RT >= 1 && RT <= kFusedMaxRT && (int8 || D != 128 || RT == 1);
}

template <int D, bool INT8, bool SC>
int launch_rt(int RT, const AttnArgs& a, dim3 grid, hipStream_t s) {
  if (a.qkv_mode) {
    if (!fused_ok(D, INT8, RT)) return COOPT_EINVAL;  // the caller checked; not reached
    const bool part = a.qkv_mode == 2;
    if constexpr (fused_ok(D, INT8, 2)) {
      if (RT == 2) {
        if (part) hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 2, SC, 2>), grid, dim3(64 * waves_for(2)), 0, s, ATTN_LEAD(a), a);
        else hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 2, SC, 1>), grid, dim3(64 * waves_for(2)), 0, s, ATTN_LEAD(a), a);
      }
    }
    if (RT == 1) {
      if (part) hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 1, SC, 2>), grid, dim3(64 * waves_for(1)), 0, s, ATTN_LEAD(a), a);
      else hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 1, SC, 1>), grid, dim3(64 * waves_for(1)), 0, s, ATTN_LEAD(a), a);
    }
    return coopt::check_launch("coopt_verify_attention_qkv");  // one split: no merge launch
  }
  switch (RT) {
    case 1: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 1, SC, 0>), grid, dim3(64 * waves_for(1)), 0, s, ATTN_LEAD(a), a); break;
    case 2: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 2, SC, 0>), grid, dim3(64 * waves_for(2)), 0, s, ATTN_LEAD(a), a); break;
    case 3: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 3, SC, 0>), grid, dim3(64 * waves_for(3)), 0, s, ATTN_LEAD(a), a); break;
    case 4: hipLaunchKernelGGL((verify_attn_kernel<D, INT8, 4, SC, 0>), grid, dim3(64 * waves_for(4)), 0, s, ATTN_LEAD(a), a); break;
    default: return COOPT_EINVAL;
  }
  int rc = coopt::check_launch("coopt_verify_attention");
  if (rc != COOPT_OK || a.max_splits <= 1) return rc;
  hipLaunchKernelGGL((merge_kernel<D>), dim3(a.Hkv, a.B), dim3(kThreads), 0, s, a);
  return coopt::check_launch("coopt_verify_attention/merge");
}

template <int D>
int launch_d(bool int8, bool sc, int RT, const AttnArgs& a, dim3 grid, hipStream_t s) {
  if (!int8) return launch_rt<D, false, false>(RT, a, grid, s);
  return sc ? launch_rt<D, true, true>(RT, a, grid, s) : launch_rt<D, true, false>(RT, a, grid, s);
}

}  // namespace

extern "C" size_t coopt_verify_attention_workspace(int B, int Hq, int Hkv, int D, int max_seqlen_q,
                                                   int max_seqlen_k) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || Hq / Hkv > kMaxRows || max_seqlen_q <= 0 ||
      max_seqlen_k <= 0)
    return 0;
  const AttnShape sh = attn_shape(B, Hq / Hkv, Hkv, max_seqlen_q, max_seqlen_k);
  if (sh.nwin > 0) return 256;  // one split per window: no partials
  return attn_ws_layout(B, Hkv, D, sh.rmax, sh.max_splits).total;
}

namespace {

// The fused epilogue's inputs (coopt_verify_attention_qkv); null for coopt_verify_attention.
struct FusedQkv {
  const void* qkv;
  int64_t qkv_tok_stride;
  const float* part;
  int ks;
  int64_t slice_stride;
  const int64_t* positions;
  const void* cos;
  const void* sin;
  int64_t table_stride;
  int max_pos;
  const int64_t* slot_mapping;
};

#define ATTN_REQUIRE(cond, msg)                              \
  do {                                                       \
    if (!(cond)) {                                           \
      coopt::set_error(std::string(who) + ": " + (msg));     \
      return COOPT_EINVAL;                                   \
    }                                                        \
  } while (0)

int verify_attention_impl(const char* who, const FusedQkv* fz, int kv_dtype, const void* q,
                          int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                          const void* v_cache, int64_t c_blk_stride, int64_t c_tok_stride,
                          int64_t c_head_stride, const void* k_scale, const void* v_scale,
                          int64_t s_blk_stride, int64_t s_tok_stride, int64_t s_head_stride,
                          const int32_t* block_table, int64_t bt_stride,
                          const int32_t* cu_seqlens_q, const int32_t* seq_lens, int B, int Hq,
                          int Hkv, int D, int block_size, int64_t num_blocks, int max_seqlen_q,
                          int max_seqlen_k, float softmax_scale, void* out, int64_t o_tok_stride,
                          int64_t o_head_stride, void* workspace, size_t workspace_bytes,
                          coopt_stream_t stream) {
  ATTN_REQUIRE(kv_dtype == COOPT_DT_BF16 || kv_dtype == COOPT_DT_I8,
               "kv_dtype must be COOPT_DT_BF16 or COOPT_DT_I8");
  ATTN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "Hq must be a multiple of Hkv");
  ATTN_REQUIRE(D == 64 || D == 128, "head_dim must be 64 or 128");
  ATTN_REQUIRE(block_size >= 16 && (block_size & (block_size - 1)) == 0,
               "block_size must be a power of two >= 16");
  ATTN_REQUIRE(max_seqlen_q > 0 && max_seqlen_k > 0, "max_seqlen_q/k must be positive");
  const int G = Hq / Hkv;
  ATTN_REQUIRE(G <= kMaxRows, "Hq/Hkv must be <= 64");
  ATTN_REQUIRE(bt_stride >= (max_seqlen_k + block_size - 1) / block_size,
               "block_table narrower than ceil(max_seqlen_k / block_size)");
  if (B == 0) return COOPT_OK;
  ATTN_REQUIRE((q || fz) && k_cache && v_cache && block_table && cu_seqlens_q && seq_lens && out,
               "null pointer");
  ATTN_REQUIRE((fz || (coopt::aligned16(q) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0)) &&
                   coopt::aligned16(out) && o_tok_stride % 8 == 0 && o_head_stride % 8 == 0,
               "q/out rows must be 16-byte aligned");
  const bool int8 = kv_dtype == COOPT_DT_I8;
  if (int8) {
    ATTN_REQUIRE(k_scale && v_scale, "INT8 KV needs k_scale and v_scale");
    ATTN_REQUIRE(coopt::aligned16(k_cache) && coopt::aligned16(v_cache) && c_blk_stride % 16 == 0 &&
                     c_tok_stride % 16 == 0 && c_head_stride % 16 == 0,
                 "INT8 cache rows must be 16-byte aligned");
  } else {
    ATTN_REQUIRE(coopt::aligned16(k_cache) && coopt::aligned16(v_cache) && c_blk_stride % 8 == 0 &&
                     c_tok_stride % 8 == 0 && c_head_stride % 8 == 0,
                 "bf16 cache rows must be 16-byte aligned");
  }
  const size_t need = coopt_verify_attention_workspace(B, Hq, Hkv, D, max_seqlen_q, max_seqlen_k);
  if (workspace_bytes < need || workspace == nullptr) {
    coopt::set_error(std::string(who) + ": workspace too small");
    return COOPT_EWORKSPACE;
  }
  ATTN_REQUIRE(num_blocks > 0, "num_blocks must be positive");
  // lanes address a page's rows with 32-bit byte offsets
  ATTN_REQUIRE(c_tok_stride > 0 && (block_size * c_tok_stride + D) * (int8 ? 1 : 2) < (int64_t{1} << 31) &&
                   (!int8 || (s_tok_stride >= 0 && block_size * s_tok_stride * 2 < (int64_t{1} << 31))),
               "cache token stride too large for one page");

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
  const AttnShape shape = attn_shape(B, G, Hkv, max_seqlen_q, max_seqlen_k);
  // grid limits: 2^32 work-items along x, 65535 blocks along z
  ATTN_REQUIRE(shape.nwin == 0 || static_cast<int64_t>(B) * shape.nwin * Hkv < (int64_t{1} << 24),
               "too many query windows for one launch");
  ATTN_REQUIRE(shape.nwin > 0 || B <= 65535, "batch must be <= 65535 sequences");
  a.rmax = shape.rmax;
  a.qwin = shape.qwin;
  a.nwin = shape.nwin;
  a.split = shape.split;
  a.max_splits = shape.max_splits;
  a.B = B;
  a.plan = shape.plan;
  const AttnWs w = attn_ws_layout(B, Hkv, D, a.rmax, a.max_splits);
  char* base = static_cast<char*>(workspace);
  a.part_ml = reinterpret_cast<float2*>(base + w.ml_off);
  a.part_o = reinterpret_cast<float*>(base + w.o_off);
  if (fz) {
    // one block per (sequence, KV head) owns that pair's rows: the epilogue cannot be shared
    // between the blocks of a split context
    ATTN_REQUIRE(fused_ok(D, int8, (a.rmax + 15) / 16),
                 "(Hq/Hkv) * max_seqlen_q must be <= 32 (<= 16 with bf16 KV at head_dim 128)");
    ATTN_REQUIRE(shape.max_splits == 1,
                 "this launch splits contexts (B * Hkv too small for max_seqlen_k); call "
                 "coopt_qkv_epilogue and coopt_verify_attention instead");
    ATTN_REQUIRE((fz->qkv != nullptr) != (fz->part != nullptr), "exactly one of qkv / part");
    ATTN_REQUIRE(!fz->part || (fz->ks >= 1 && fz->ks <= kQkvMaxSlices && coopt::aligned16(fz->part) &&
                               fz->slice_stride % 4 == 0),
                 "part needs 1 <= ks <= 4 slices, 16-byte aligned");
    ATTN_REQUIRE(!fz->qkv || (coopt::aligned16(fz->qkv) && fz->qkv_tok_stride % 8 == 0 &&
                              fz->qkv_tok_stride >= static_cast<int64_t>(Hq + 2 * Hkv) * D),
                 "qkv rows must be 16-byte aligned and hold (Hq + 2 Hkv) * D elements");
    ATTN_REQUIRE(fz->positions && fz->cos && fz->sin && fz->slot_mapping, "null pointer");
    ATTN_REQUIRE(coopt::aligned16(fz->cos) && coopt::aligned16(fz->sin) && fz->table_stride % 8 == 0 &&
                     fz->table_stride >= D / 2 && fz->max_pos > 0,
                 "cos/sin tables must be 16-byte aligned rows of >= D/2 bf16");
    ATTN_REQUIRE(fz->table_stride < (int64_t{1} << 31) && (num_blocks << shift) / block_size == num_blocks,
                 "table stride or pool size out of range");
    a.qkv_mode = fz->part ? 2 : 1;
    a.qkv_src = fz->part ? static_cast<const void*>(fz->part) : fz->qkv;
    a.qkv_stride = fz->part ? fz->slice_stride : fz->qkv_tok_stride;
    a.qkv_ks = fz->ks;
    a.pos = fz->positions;
    a.cos = static_cast<const uint16_t*>(fz->cos);
    a.sin = static_cast<const uint16_t*>(fz->sin);
    a.tab_stride = static_cast<int>(fz->table_stride);
    a.max_pos = fz->max_pos;
    a.slots = fz->slot_mapping;
  }
  coopt::clear_error();

  const int RT = (a.rmax + 15) / 16;
  const dim3 grid = shape.nwin > 0 ? dim3(B * shape.nwin * Hkv)
                    : (shape.plan ? dim3(B * Hkv) : dim3(a.max_splits, Hkv, B));
  auto s = static_cast<hipStream_t>(stream);
  // scale caches with consecutive tokens adjacent and 8-byte aligned groups of four
  const bool sc = int8 && s_tok_stride == 1 && s_blk_stride % 4 == 0 && s_head_stride % 4 == 0 &&
                  (reinterpret_cast<uintptr_t>(k_scale) & 7u) == 0 &&
                  (reinterpret_cast<uintptr_t>(v_scale) & 7u) == 0;
  return D == 128 ? launch_d<128>(int8, sc, RT, a, grid, s) : launch_d<64>(int8, sc, RT, a, grid, s);
}

#undef ATTN_REQUIRE

}  // namespace

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
  return verify_attention_impl("coopt_verify_attention", nullptr, kv_dtype, q, q_tok_stride,
                               q_head_stride, k_cache, v_cache, c_blk_stride, c_tok_stride,
                               c_head_stride, k_scale, v_scale, s_blk_stride, s_tok_stride,
                               s_head_stride, block_table, bt_stride, cu_seqlens_q, seq_lens, B,
                               Hq, Hkv, D, block_size, num_blocks, max_seqlen_q, max_seqlen_k,
                               softmax_scale, out, o_tok_stride, o_head_stride, workspace,
                               workspace_bytes, stream);
}

extern "C" int coopt_verify_attention_qkv_supported(int kv_dtype, int B, int Hq, int Hkv, int D,
                                                    int max_seqlen_q, int max_seqlen_k) {
  if (kv_dtype != COOPT_DT_BF16 && kv_dtype != COOPT_DT_I8) return 0;
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || max_seqlen_q <= 0 || max_seqlen_k <= 0) return 0;
  if (D != 64 && D != 128) return 0;
  const int G = Hq / Hkv;
  if (static_cast<int64_t>(G) * max_seqlen_q > kMaxRows) return 0;
  if (!fused_ok(D, kv_dtype == COOPT_DT_I8, (G * max_seqlen_q + 15) / 16)) return 0;
  return attn_shape(B, G, Hkv, max_seqlen_q, max_seqlen_k).max_splits == 1 ? 1 : 0;
}

extern "C" int coopt_verify_attention_qkv(
    int kv_dtype, const void* qkv, int64_t qkv_tok_stride, const float* part, int ks,
    int64_t slice_stride, const int64_t* positions, const void* cos, const void* sin,
    int64_t table_stride, int max_pos, const int64_t* slot_mapping, void* k_cache, void* v_cache,
    int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride, void* k_scale,
    void* v_scale, int64_t s_blk_stride, int64_t s_tok_stride, int64_t s_head_stride,
    const int32_t* block_table, int64_t bt_stride, const int32_t* cu_seqlens_q,
    const int32_t* seq_lens, int B, int Hq, int Hkv, int D, int block_size, int64_t num_blocks,
    int max_seqlen_q, int max_seqlen_k, float softmax_scale, void* out, int64_t o_tok_stride,
    int64_t o_head_stride, void* workspace, size_t workspace_bytes, coopt_stream_t stream) {
  const FusedQkv fz{qkv, qkv_tok_stride, part, ks, slice_stride, positions, cos, sin,
                    table_stride, max_pos, slot_mapping};
  return verify_attention_impl("coopt_verify_attention_qkv", &fz, kv_dtype, nullptr, 0, 0,
                               k_cache, v_cache, c_blk_stride, c_tok_stride, c_head_stride,
                               k_scale, v_scale, s_blk_stride, s_tok_stride, s_head_stride,
                               block_table, bt_stride, cu_seqlens_q, seq_lens, B, Hq, Hkv, D,
                               block_size, num_blocks, max_seqlen_q, max_seqlen_k, softmax_scale,
                               out, o_tok_stride, o_head_stride, workspace, workspace_bytes,
                               stream);
}
