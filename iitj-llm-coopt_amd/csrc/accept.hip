// Fused speculative acceptance: vocab-wide softmax of target and draft rows, the p/q accept
// test, first rejection, the max(0, p - q) residual and inverse-CDF resampling, for a whole
// batch.  Semantics: engine/spec_decode.py:20-49 (sampling) and :30-35 (greedy), looped over
// the batch at engine/engine.py:421-446, with the uniforms explicit.
//
// Launches (each reads what the previous one wrote; no cross-block fences or counters):
//   1. row_stats_kernel, grid (chunk, row slot, sequence): one chunk of one row per block --
//      max of x/T and an fp64 sum of exp(x/T - max) (sampling), or max and first argmax
//      (greedy).  Full chunks are read with unconditional 16-byte loads, all issued before use.
//      Sampling: the block whose chunk holds the row's draft token also stores x/T there.
//   2. greedy_kernel, grid (sequence): combines the argmax partials and applies the prefix
//      rule.  -- or, sampling --
//      decide_kernel, grid (chunk, sequence): every block combines its sequence's row
//      statistics (one chunk partial per thread, lane groups reducing each row) and wave 0
//      makes the accept decision with a ballot over the drafts, all from one round of
//      independent loads; then the block sums the resampling weights w_j of its chunk.
//      Block 0 of each sequence publishes the accepted prefix and the decision.
//   3. select_kernel, grid (sequence): finds the chunk where the cumulative weight crosses
//      u * sum(w), scans it and writes the emitted token.
// Per-block reductions and prefix sums in fp64 run on DPP / permlane lane exchanges.
//
// Numerics.  Row maxima are exact and sum(exp) is accumulated in fp64.  The probabilities at
// the draft tokens, which decide acceptance, are formed with an fp64 exp and rounded once to
// fp32, so p_i[d_i] / q_i[d_i] agree with an exactly rounded fp32 softmax except within an
// ulp of a rounding boundary.  The vocab-wide terms use exp2(fma(x, log2 e, -max log2 e))
// (relative error < 1e-6); cumulative weights are fp64 sums of fp32 w_j.
#include <math.h>

#include <mutex>
#include <string>

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 64;                    // elements a phase-1 thread keeps in VGPRs
constexpr int kMaxChunk = kThreads * kMaxPerThread;  // 16384
constexpr int kMinChunk = 1024;
constexpr int kMaxSlots = 2 * 64 + 1;                // 2 * gamma_max + 1 rows per sequence
constexpr float kLog2e = 1.4426950408889634f;

enum : int { kModeResidual = 0, kModeBonus = 1 };

struct Partial1 {  // per (sequence, row slot, chunk)
  float m;         // chunk max of x/T (greedy: max logit)
  int idx;         // greedy: first index of the max
  double s;        // sum of exp(x/T - m) over the chunk
};
struct RowStat {
  float m;
  int argmax;
  double s;
};
struct Decision {
  int k;
  int mode;
  float margin;
  int pad;
  RowStat rt, rq;  // statistics of the target / draft row the token is drawn from
};
struct Partial2 {
  double w;  // sum of resampling weights over the chunk
  double p;  // sum of target probabilities (fallback when the residual is all zero)
};

struct Layout {
  int nch1, chunk1, nch2, chunk2;
};

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ inline int imax(int a, int b) { return a > b ? a : b; }
__host__ __device__ inline int imin(int a, int b) { return a < b ? a : b; }

// Chunking is a pure function of (B, gamma_max, V) so the workspace size can be computed
// without the data.  Chunks are multiples of 8 elements; at most kThreads resampling chunks.
// Launch 1 aims at ~512 blocks, i.e. as many elements per thread (up to kMaxPerThread, all
// loads in flight at once) as the batch allows: at B = 8 that measured 28 us per call
// against 34 us with 2048 smaller blocks.
// gamma_max = 0 (a plain draw): chunks of at most kDrawChunk elements, the chunk the draw
// block of launch 2 scans in registers (kDrawG 8-element groups a thread).
constexpr int kDrawG = 4;
constexpr int kDrawChunk = kThreads * 8 * kDrawG;  // 8192

__host__ __device__ inline Layout make_layout(int B, int gmax, int V) {
  Layout L;
  const int rows = B * (2 * gmax + 1);
  int nch = ceil_div(512, rows > 0 ? rows : 1);
  nch = imax(nch, ceil_div(V, gmax == 0 ? kDrawChunk : kMaxChunk));
  nch = imin(nch, imax(1, ceil_div(V, kMinChunk)));
  L.chunk1 = ceil_div(ceil_div(V, nch), 8) * 8;
  L.nch1 = ceil_div(V, L.chunk1);
  int nch2 = ceil_div(1024, B > 0 ? B : 1);
  nch2 = imax(1, imin(nch2, imin(kThreads, ceil_div(V, kMinChunk))));
  L.chunk2 = ceil_div(ceil_div(V, nch2), 8) * 8;
  L.nch2 = ceil_div(V, L.chunk2);
  return L;
}

struct Workspace {
  Partial1* part1;  // [B][2*gmax+1][nch1]
  Decision* dec;    // [B]
  Partial2* part2;  // [B][nch2]
  float* tokx;      // [B][2*gmax+1]: x/T at the row's draft token (launch 1 -> launch 2)
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Lays the workspace out from `base` (0 to only measure it); returns its size in bytes.
__host__ __device__ inline size_t carve(Workspace* w, uintptr_t base, int B, int gmax, const Layout& L) {
  const int slots = 2 * gmax + 1;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const uintptr_t p = base + off;
    off += align256(bytes);
    return p;
  };
  w->part1 = reinterpret_cast<Partial1*>(take(sizeof(Partial1) * B * slots * L.nch1));
  w->dec = reinterpret_cast<Decision*>(take(sizeof(Decision) * B));
  w->part2 = reinterpret_cast<Partial2*>(take(sizeof(Partial2) * B * L.nch2));
  w->tokx = reinterpret_cast<float*>(take(sizeof(float) * B * slots));
  return off;
}

struct Args {
  const void* tgt;
  int64_t tgt_stride;
  const int32_t* tgt_row0;
  const void* drf;
  int64_t drf_stride;
  const int32_t* drf_row0;
  const int32_t* dtok;
  const int32_t* gam;
  const float* u_acc;
  const float* u_res;
  int32_t* acc_len;
  int32_t* out_tok;
  float* margin;
  float inv_t;
  int draft_probs;
  int vec_t, vec_d;  // rows may be read with 16-byte loads
  int B, gmax, V;
  Layout L;
  Workspace ws;
};

__device__ __forceinline__ int gamma_of(const Args& a, int b) {
  return a.gam ? min(max(a.gam[b], 0), a.gmax) : a.gmax;
}
__device__ __forceinline__ int64_t tgt_row(const Args& a, int b, int i) {
  return (a.tgt_row0 ? static_cast<int64_t>(a.tgt_row0[b]) : static_cast<int64_t>(b) * (a.gmax + 1)) + i;
}
__device__ __forceinline__ int64_t drf_row(const Args& a, int b, int i) {
  return (a.drf_row0 ? static_cast<int64_t>(a.drf_row0[b]) : static_cast<int64_t>(b) * a.gmax) + i;
}

template <bool BF16>
__device__ __forceinline__ float ld(const void* base, int64_t row, int64_t stride, int j) {
  if constexpr (BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(base)[row * stride + j]);
  } else {
    return static_cast<const float*>(base)[row * stride + j];
  }
}

// Loads 8 consecutive elements starting at j (16 bytes of bf16, or two 16-byte fp32 loads).
template <bool BF16>
__device__ __forceinline__ void ld8(const void* base, int64_t row, int64_t stride, int j, float* v) {
  if constexpr (BF16) {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + row * stride + j);
    const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __uint_as_float(w4[e] << 16);
      v[2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + row * stride + j);
    const float4 r0 = p[0], r1 = p[1];
    v[0] = r0.x; v[1] = r0.y; v[2] = r0.z; v[3] = r0.w;
    v[4] = r1.x; v[5] = r1.y; v[6] = r1.z; v[7] = r1.w;
  }
}

// Block-wide reductions over kThreads threads (4 waves) through LDS.
__device__ __forceinline__ float block_max(float v, float* sh) {
  v = wave_max_f32(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum(double v, double* sh) {
  v = wave_sum_f64(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  const double r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return r;
}

// (value, index) argmax with first-index tie break.
__device__ __forceinline__ void amax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

// exp(x - m) for the vocab-wide terms: one fma and v_exp_f32.
__device__ __forceinline__ float exp_shift(float x, float m_l2) {
  return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -m_l2));
}

// Accurate p = exp(x' - m) / s rounded once to fp32 (x' = fl32(x * inv_t)).
__device__ __forceinline__ float prob_at(float xs, float m, double s) {
  return static_cast<float>(exp(static_cast<double>(xs) - static_cast<double>(m)) / s);
}

// ---------------------------------------------------------------------------------------
// Launch 1: per-chunk row statistics.
// ---------------------------------------------------------------------------------------
template <bool BF16, bool GREEDY>
__global__ __launch_bounds__(kThreads) void row_stats_kernel(Args a) {
  __shared__ float shf[4];
  __shared__ double shd[4];
  __shared__ float shv[4];
  __shared__ int shi[4];
  const int c = blockIdx.x, slot = blockIdx.y, b = blockIdx.z;
  const int g = gamma_of(a, b);
  const bool is_draft = slot > a.gmax;
  const int i = is_draft ? slot - a.gmax - 1 : slot;
  if (!is_draft && i > g) return;
  if (is_draft && (GREEDY || a.draft_probs || i >= g)) return;

  const void* base = is_draft ? a.drf : a.tgt;
  const int64_t stride = is_draft ? a.drf_stride : a.tgt_stride;
  const int64_t row = is_draft ? drf_row(a, b, i) : tgt_row(a, b, i);
  // Sampling: the draft token this row is tested at (draft i and target i < g; the bonus
  // row g has none).  The block whose chunk holds it hands x/T there to launch 2.
  const int tok = (!GREEDY && (is_draft || i < g)) ? a.dtok[static_cast<int64_t>(b) * a.gmax + i] : -1;
  const int lo = c * a.L.chunk1;
  const int hi = min(a.V, lo + a.L.chunk1);
  const int tid = threadIdx.x;
  // Element (it, e) of this thread is lo + (it * kThreads + tid) * 8 + e.  Chunks are
  // multiples of 8, so in a full chunk a group is either wholly inside or wholly past hi.
  const bool full = (is_draft ? a.vec_d : a.vec_t) != 0 && hi - lo == a.L.chunk1;
  float vals[kMaxPerThread];
#pragma unroll
  for (int it = 0; it < kMaxPerThread / 8; ++it) {
    const int j0 = lo + (it * kThreads + tid) * 8;
    if (full && j0 < hi) {
      ld8<BF16>(base, row, stride, j0, vals + it * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vals[it * 8 + e] = (j0 + e < hi) ? ld<BF16>(base, row, stride, j0 + e) : -INFINITY;
    }
  }

  Partial1 part;
  if constexpr (GREEDY) {
    float v = -INFINITY;
    int idx = 0x7fffffff;
#pragma unroll
    for (int it = 0; it < kMaxPerThread / 8; ++it)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = lo + (it * kThreads + tid) * 8 + e;
        if (j < hi) amax_merge(v, idx, vals[it * 8 + e], j);
      }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const float ov = __shfl_xor(v, m, 64);
      const int oi = __shfl_xor(idx, m, 64);
      amax_merge(v, idx, ov, oi);
    }
    const int w = tid >> 6;
    if ((tid & 63) == 0) {
      shv[w] = v;
      shi[w] = idx;
    }
    __syncthreads();
    v = shv[0];
    idx = shi[0];
    for (int q = 1; q < 4; ++q) amax_merge(v, idx, shv[q], shi[q]);
    part.m = v;
    part.idx = idx;
    part.s = 0.0;
  } else {
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < kMaxPerThread; ++e) {
      vals[e] *= a.inv_t;
      m = fmaxf(m, vals[e]);
    }
    if (tok >= lo && tok < hi) {  // uniform; one thread holds element tok
      const int t = (tok - lo) >> 3;
      if (tid == t % kThreads) {
        const int pos = (t / kThreads) * 8 + ((tok - lo) & 7);
        float x = 0.0f;
#pragma unroll
        for (int e = 0; e < kMaxPerThread; ++e) x = (e == pos) ? vals[e] : x;
        a.ws.tokx[static_cast<int64_t>(b) * (2 * a.gmax + 1) + slot] = x;
      }
    }
    m = block_max(m, shf);
    double s = 0.0;
    if (m > -INFINITY) {
      const float m_l2 = m * kLog2e;
#pragma unroll
      for (int it = 0; it < kMaxPerThread / 8; ++it) {
        float acc = 0.0f;  // 8 terms <= 1 each in fp32, then fp64
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += exp_shift(vals[it * 8 + e], m_l2);
        s += static_cast<double>(acc);
      }
    }
    s = block_sum(s, shd);
    part.m = m;
    part.idx = -1;
    part.s = s;
  }
  if (tid == 0) a.ws.part1[(static_cast<int64_t>(b) * (2 * a.gmax + 1) + slot) * a.L.nch1 + c] = part;
}

// Combines the chunk partials of row slot `slot` of sequence b (chunk order).
__device__ __forceinline__ RowStat combine_row(const Args& a, int b, int slot, bool greedy) {
  const Partial1* p = a.ws.part1 + (static_cast<int64_t>(b) * (2 * a.gmax + 1) + slot) * a.L.nch1;
  RowStat rs;
  if (greedy) {
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int c = 0; c < a.L.nch1; ++c) amax_merge(v, idx, p[c].m, p[c].idx);
    rs.m = v;
    rs.argmax = idx;
    rs.s = 0.0;
  } else {
    float m = -INFINITY;
    for (int c = 0; c < a.L.nch1; ++c) m = fmaxf(m, p[c].m);
    double s = 0.0;
    for (int c = 0; c < a.L.nch1; ++c) {
      const Partial1 q = p[c];
      if (q.s > 0.0) s += q.s * exp(static_cast<double>(q.m) - static_cast<double>(m));
    }
    rs.m = m;
    rs.argmax = -1;
    rs.s = s;
  }
  return rs;
}

// Sampling statistics of every row slot of sequence b, one wave per row: lanes read the chunk
// partials in parallel, then (max, sum * exp(m_c - max)) reduce across the wave.  The sum
// follows the chunk order of combine_row's serial loop only up to fp64 rounding.
__device__ __forceinline__ void combine_rows_waves(const Args& a, int b, int nrow_t, int nrow_d,
                                                   RowStat* rows) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nrows = nrow_t + nrow_d;
  for (int r = wave; r < nrows; r += kThreads / 64) {
    const int slot = r < nrow_t ? r : (a.gmax + 1) + (r - nrow_t);
    const Partial1* p = a.ws.part1 + (static_cast<int64_t>(b) * (2 * a.gmax + 1) + slot) * a.L.nch1;
    float m = -INFINITY;
    for (int c = lane; c < a.L.nch1; c += 64) m = fmaxf(m, p[c].m);
    m = wave_max_f32(m);
    double s = 0.0;
    for (int c = lane; c < a.L.nch1; c += 64) {
      const Partial1 q = p[c];
      if (q.s > 0.0) s += q.s * exp(static_cast<double>(q.m) - static_cast<double>(m));
    }
    s = wave_sum_f64(s);
    if (lane == 0) {
      rows[slot].m = m;
      rows[slot].argmax = -1;
      rows[slot].s = s;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Launch 2 (greedy): argmax prefix rule, one block per sequence.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void greedy_kernel(Args a) {
  __shared__ int argm[kMaxSlots];
  const int b = blockIdx.x;
  const int g = gamma_of(a, b);
  // row slot i <= g by wave i % 4: lanes merge chunks lane, lane + 64, .. in order, then the
  // wave merges lanes (first index on ties, as a serial merge in chunk order gives)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = wave; i <= g; i += kThreads / 64) {
    const Partial1* p = a.ws.part1 + (static_cast<int64_t>(b) * (2 * a.gmax + 1) + i) * a.L.nch1;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int c = lane; c < a.L.nch1; c += 64) amax_merge(v, idx, p[c].m, p[c].idx);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const float ov = __shfl_xor(v, m, 64);
      const int oi = __shfl_xor(idx, m, 64);
      amax_merge(v, idx, ov, oi);
    }
    if (lane == 0) argm[i] = idx;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  const int32_t* d = a.dtok + static_cast<int64_t>(b) * a.gmax;
  int32_t* out = a.out_tok + static_cast<int64_t>(b) * (a.gmax + 1);
  int k = g;
  for (int i = 0; i < g; ++i) {
    if (argm[i] != d[i]) {
      k = i;
      break;
    }
  }
  for (int i = 0; i < k; ++i) out[i] = d[i];
  out[k] = argm[k];
  for (int i = k + 1; i <= a.gmax; ++i) out[i] = -1;
  a.acc_len[b] = k;
  if (a.margin) a.margin[b] = INFINITY;
}

// Resampling weights of up to 8 elements j.. (bit-identical wherever evaluated).
template <bool BF16>
struct WeightRow {
  const Args* a;
  int64_t trow, drow;
  int mode;
  float mt_l2, mq_l2;
  double inv_st, inv_sq;

  __device__ __forceinline__ void at(int j, int n, bool vec, float* w, float* p) const {
    float xt[8], xq[8];
    if (vec) {
      ld8<BF16>(a->tgt, trow, a->tgt_stride, j, xt);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xt[e] = e < n ? ld<BF16>(a->tgt, trow, a->tgt_stride, j + e) : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      p[e] = static_cast<float>(static_cast<double>(exp_shift(xt[e] * a->inv_t, mt_l2)) * inv_st);
    if (mode == kModeBonus) {
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = p[e];
      return;
    }
    float q[8];
    if (a->draft_probs) {
      const float* qr = static_cast<const float*>(a->drf) + drow * a->drf_stride;
      if (vec) {
        const float4 q0 = *reinterpret_cast<const float4*>(qr + j);
        const float4 q1 = *reinterpret_cast<const float4*>(qr + j + 4);
        q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w;
        q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = e < n ? qr[j + e] : 0.0f;
      }
    } else {
      if (vec) {
        ld8<BF16>(a->drf, drow, a->drf_stride, j, xq);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xq[e] = e < n ? ld<BF16>(a->drf, drow, a->drf_stride, j + e) : -INFINITY;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        q[e] = static_cast<float>(static_cast<double>(exp_shift(xq[e] * a->inv_t, mq_l2)) * inv_sq);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = fmaxf(p[e] - q[e], 0.0f);
  }

  // at() for a full vectorised group (j + 8 <= V) in two halves: load() issues the group's
  // loads and finish() forms w and p from them with at()'s arithmetic, so a caller can have
  // several groups' loads in flight before the first use.
  struct Raw {
    float xt[8], xq[8];
  };
  __device__ __forceinline__ void load(int j, Raw& r) const {
    ld8<BF16>(a->tgt, trow, a->tgt_stride, j, r.xt);
    if (mode == kModeBonus) return;
    if (a->draft_probs) {
      const float4* qp = reinterpret_cast<const float4*>(static_cast<const float*>(a->drf) + drow * a->drf_stride + j);
      const float4 q0 = qp[0], q1 = qp[1];
      r.xq[0] = q0.x; r.xq[1] = q0.y; r.xq[2] = q0.z; r.xq[3] = q0.w;
      r.xq[4] = q1.x; r.xq[5] = q1.y; r.xq[6] = q1.z; r.xq[7] = q1.w;
    } else {
      ld8<BF16>(a->drf, drow, a->drf_stride, j, r.xq);
    }
  }
  __device__ __forceinline__ void finish(const Raw& r, float* w, float* p) const {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      p[e] = static_cast<float>(static_cast<double>(exp_shift(r.xt[e] * a->inv_t, mt_l2)) * inv_st);
    if (mode == kModeBonus) {
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = p[e];
      return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = a->draft_probs
                          ? r.xq[e]
                          : static_cast<float>(static_cast<double>(exp_shift(r.xq[e] * a->inv_t, mq_l2)) * inv_sq);
      w[e] = fmaxf(p[e] - q, 0.0f);
    }
  }
};

// trow0 / drow0: tgt_row(a, b, 0) / drf_row(a, b, 0), read by the caller ahead of the decision.
template <bool BF16>
__device__ __forceinline__ WeightRow<BF16> make_weight_row(const Args& a, int64_t trow0, int64_t drow0,
                                                           const Decision& dec) {
  WeightRow<BF16> wr;
  wr.a = &a;
  wr.mode = dec.mode;
  wr.trow = trow0 + dec.k;
  wr.drow = dec.mode == kModeResidual ? drow0 + dec.k : 0;
  wr.mt_l2 = dec.rt.m * kLog2e;
  wr.mq_l2 = dec.rq.m * kLog2e;
  wr.inv_st = 1.0 / dec.rt.s;
  wr.inv_sq = dec.mode == kModeResidual && !a.draft_probs ? 1.0 / dec.rq.s : 0.0;
  return wr;
}

// Max / sum over aligned groups of G = 8 or 16 consecutive lanes (DPP, every lane of a group
// gets the same bits).
template <int G>
__device__ __forceinline__ float group_max_f32(float v) {
  v = fmaxf(v, dpp_f32<dpp::kXor1>(v));
  v = fmaxf(v, dpp_f32<dpp::kXor2>(v));
  v = fmaxf(v, dpp_f32<dpp::kRowHalfMirror>(v));
  if constexpr (G == 16) v = fmaxf(v, dpp_f32<dpp::kRowMirror>(v));
  return v;
}
template <int G>
__device__ __forceinline__ double group_sum_f64(double v) {
  v += dpp_f64<dpp::kXor1>(v);
  v += dpp_f64<dpp::kXor2>(v);
  v += dpp_f64<dpp::kRowHalfMirror>(v);
  if constexpr (G == 16) v += dpp_f64<dpp::kRowMirror>(v);
  return v;
}

// Sampling statistics of every row slot of sequence b when a row has at most G chunks: thread
// t takes chunk t % G of slot s0 + t / G (one load each, all slots at once, whatever g is), and
// the G lanes of a slot reduce (max, sum * exp(m_c - max)) together.  load_group issues the
// load; reduce_group uses it.
struct ChunkStat {
  float m;
  double s;
};
template <int G>
__device__ __forceinline__ ChunkStat load_group(const Args& a, int b, int s0) {
  const int slots = 2 * a.gmax + 1;
  const int slot = s0 + static_cast<int>(threadIdx.x) / G, c = threadIdx.x % G;
  ChunkStat q{-INFINITY, 0.0};
  if (slot < slots && c < a.L.nch1) {
    const Partial1& p = a.ws.part1[(static_cast<int64_t>(b) * slots + slot) * a.L.nch1 + c];
    q.m = p.m;
    q.s = p.s;
  }
  return q;
}
template <int G>
__device__ __forceinline__ void reduce_group(const Args& a, ChunkStat q, int s0, RowStat* rows) {
  const int slot = s0 + static_cast<int>(threadIdx.x) / G;
  const float mx = group_max_f32<G>(q.m);
  const double t = q.s * exp(static_cast<double>(q.m) - static_cast<double>(mx));
  const double sum = group_sum_f64<G>(q.s > 0.0 ? t : 0.0);  // empty chunks add nothing
  if (threadIdx.x % G == 0 && slot < 2 * a.gmax + 1) {
    rows[slot].m = mx;
    rows[slot].argmax = -1;
    rows[slot].s = sum;
  }
}

// The accept decision of sequence b, made by wave 0 (threadIdx.x < 64) from the row statistics
// in `rows` (LDS).  Lane i holds draft i's token, uniform and the logits at the token (launch 1
// captured them); their loads are issued by the caller before the rows are combined.
struct TokenLane {
  int tok;
  float xt, xq, u;
};
__device__ __forceinline__ TokenLane load_token_lane(const Args& a, int b) {
  const int lane = threadIdx.x;
  const int64_t sb = static_cast<int64_t>(b) * (2 * a.gmax + 1);
  TokenLane t{-1, 0.0f, 0.0f, 0.0f};
  if (lane < a.gmax) {
    t.tok = a.dtok[static_cast<int64_t>(b) * a.gmax + lane];
    t.u = a.u_acc[static_cast<int64_t>(b) * a.gmax + lane];
    t.xt = a.ws.tokx[sb + lane];
    if (!a.draft_probs) t.xq = a.ws.tokx[sb + a.gmax + 1 + lane];
  }
  return t;
}

__device__ __forceinline__ Decision decide_wave(const Args& a, int b, int g, TokenLane t,
                                                const RowStat* rows, bool publish) {
  const int lane = threadIdx.x;
  const int tok = t.tok;
  const float u = t.u;
  float mt = -INFINITY, mq = -INFINITY;
  double st = 0.0, sq = 0.0;
  if (lane < g) {
    mt = rows[lane].m;
    st = rows[lane].s;
    if (!a.draft_probs) {
      mq = rows[a.gmax + 1 + lane].m;
      sq = rows[a.gmax + 1 + lane].s;
    }
  }
  const float xt = t.xt;
  float xq = t.xq;
  const bool live = lane < g;
  const bool valid = tok >= 0 && tok < a.V;
  if (a.draft_probs && live && valid) xq = static_cast<const float*>(a.drf)[drf_row(a, b, lane) * a.drf_stride + tok];
  float ratio = 0.0f;
  if (live) {
    // an out-of-vocabulary draft token has p = 0, so it is rejected
    const float p = valid ? prob_at(xt, mt, st) : 0.0f;
    const float q = !valid ? 1.0f : (a.draft_probs ? xq : prob_at(xq, mq, sq));
    ratio = fminf(p / fmaxf(q, 1e-20f), 1.0f);
  }
  // k = the first i with u_i >= ratio_i; margin over the tests made up to and including it
  const uint64_t rej = __ballot(live && u >= ratio);
  const int k = rej ? __builtin_ctzll(rej) : g;
  const float mg = wave_min_f32_dpp((live && lane <= k) ? fabsf(u - ratio) : INFINITY);
  Decision d;
  d.k = k;
  d.mode = k < g ? kModeResidual : kModeBonus;
  d.margin = mg;
  d.pad = 0;
  // field by field from scalar reads (a whole-struct copy through the pointer went to scratch)
  const int kq = (d.mode == kModeResidual && !a.draft_probs) ? a.gmax + 1 + k : k;
  d.rt.m = rows[k].m;
  d.rt.argmax = -1;
  d.rt.s = rows[k].s;
  d.rq.m = rows[kq].m;
  d.rq.argmax = -1;
  d.rq.s = rows[kq].s;
  if (publish) {
    int32_t* out = a.out_tok + static_cast<int64_t>(b) * (a.gmax + 1);
    for (int i = lane; i <= a.gmax; i += 64) {
      if (i < k) out[i] = tok;  // i < k <= 63: i == lane, whose tok is d_i
      else if (i > k) out[i] = -1;
    }
    if (lane == 0) {
      a.ws.dec[b] = d;
      a.acc_len[b] = k;
    }
  }
  return d;
}

// ---------------------------------------------------------------------------------------
// Launch 2 (sampling): accept decision (made again by every block of the sequence, from the
// same data, so identically) and the chunk sums of the resampling weights.
// ---------------------------------------------------------------------------------------
template <bool BF16, int LC>
__global__ __launch_bounds__(kThreads) void decide_kernel(Args a) {
  __shared__ RowStat rows[kMaxSlots];
  __shared__ Decision sdec;
  __shared__ double shw[4], shp[4];
  const int c = blockIdx.x, b = blockIdx.y;
  const int g = gamma_of(a, b);
  const int64_t trow0 = tgt_row(a, b, 0), drow0 = drf_row(a, b, 0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  TokenLane tl{-1, 0.0f, 0.0f, 0.0f};
  if constexpr (LC == 0) {
    if (wave == 0) tl = load_token_lane(a, b);
    combine_rows_waves(a, b, g + 1, a.draft_probs ? 0 : g, rows);
  } else {
    // the first pass's partial loads, then wave 0's token loads, then the first use
    ChunkStat q = load_group<LC>(a, b, 0);
    if (wave == 0) tl = load_token_lane(a, b);
    reduce_group<LC>(a, q, 0, rows);
    for (int s0 = kThreads / LC; s0 < 2 * a.gmax + 1; s0 += kThreads / LC)
      reduce_group<LC>(a, load_group<LC>(a, b, s0), s0, rows);
  }
  __syncthreads();
  if (wave == 0) {
    const Decision d = decide_wave(a, b, g, tl, rows, c == 0);
    if (lane == 0) sdec = d;
  }
  __syncthreads();
  const Decision dec = sdec;
  const WeightRow<BF16> wr = make_weight_row<BF16>(a, trow0, drow0, dec);
  const int lo = c * a.L.chunk2;
  const int hi = min(a.V, lo + a.L.chunk2);
  const bool vec = a.vec_t && (dec.mode == kModeBonus || a.vec_d);
  double sw = 0.0, sp = 0.0;
  auto add = [&](const float* w, const float* p, int n) {
    float fw = 0.0f, fp = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (e < n) {
        fw += w[e];
        fp += p[e];
      }
    }
    sw += static_cast<double>(fw);
    sp += static_cast<double>(fp);
  };
  // Two groups per pass, in the order of a one-group loop.  When both are full the second
  // group's loads are issued before the first group is used (its index falls back to the
  // first group's past the chunk end, so the load is unconditional and in bounds).
  constexpr int kStep = kThreads * 8;
  for (int j = lo + tid * 8; j < hi; j += 2 * kStep) {
    const int j1 = j + kStep;
    const bool has1 = j1 < hi;
    float w[8], p[8];
    if (vec && hi - j >= 8 && (!has1 || hi - j1 >= 8)) {
      typename WeightRow<BF16>::Raw r0, r1;
      wr.load(j, r0);
      wr.load(has1 ? j1 : j, r1);
      wr.finish(r0, w, p);
      add(w, p, 8);
      if (has1) {
        wr.finish(r1, w, p);
        add(w, p, 8);
      }
    } else {
      const int n = min(8, hi - j);
      wr.at(j, n, vec && n == 8, w, p);
      add(w, p, n);
      if (has1) {
        const int n1 = min(8, hi - j1);
        wr.at(j1, n1, vec && n1 == 8, w, p);
        add(w, p, n1);
      }
    }
  }
  sw = wave_sum_f64_dpp(sw);
  sp = wave_sum_f64_dpp(sp);
  if (lane == 0) {
    shw[wave] = sw;
    shp[wave] = sp;
  }
  __syncthreads();
  if (tid == 0) {
    Partial2 pp;
    pp.w = (shw[0] + shw[1]) + (shw[2] + shw[3]);
    pp.p = (shp[0] + shp[1]) + (shp[2] + shp[3]);
    a.ws.part2[static_cast<int64_t>(b) * a.L.nch2 + c] = pp;
  }
}

// Inclusive block scan of one fp64 value per thread (4 waves): the wave scans, then the
// totals of the waves before this one added in wave order.  excl = the previous thread's
// inclusive value, bit for bit (+0.0 for thread 0); total = thread kThreads-1's.  sh[4] must
// not be rewritten before every thread has returned.
__device__ __forceinline__ double block_scan_f64(double v, double* sh, double& excl, double& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  double wex;
  const double wincl = wave_incl_scan_f64(v, wex);
  if (lane == 63) sh[w] = wincl;
  __syncthreads();
  double off = 0.0;
  for (int q = 0; q < w; ++q) off += sh[q];
  total = ((sh[0] + sh[1]) + sh[2]) + sh[3];  // == the fold off + wincl of thread kThreads-1
  excl = lane == 0 ? off : off + wex;
  return off + wincl;
}

// ---------------------------------------------------------------------------------------
// Launch 3 (sampling): inverse-CDF draw, one block per sequence.
// ---------------------------------------------------------------------------------------
template <bool BF16>
__global__ __launch_bounds__(kThreads) void select_kernel(Args a) {
  __shared__ double shs1[4], shs2[4], shs3[4];
  __shared__ double csum[kThreads];
  __shared__ int sh_cross[4], sh_lastm[4];
  __shared__ int sh_tok_min;
  __shared__ float sh_margin;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const Decision dec = a.ws.dec[b];
  const Partial2* P = a.ws.part2 + static_cast<int64_t>(b) * a.L.nch2;
  double wv = 0.0, pv = 0.0;
  if (tid < a.L.nch2) {  // nch2 <= kThreads by construction
    wv = P[tid].w;
    pv = P[tid].p;
  }
  const float ures = a.u_res[b];
  const WeightRow<BF16> wr = make_weight_row<BF16>(a, tgt_row(a, b, 0), drf_row(a, b, 0), dec);
  if (tid == 0) {
    sh_tok_min = 0x7fffffff;
    sh_margin = 0.0f;
  }
  // Chunk sums -> inclusive prefix sums, one chunk per thread (fp64).  The resampling weights
  // are used unless the residual sums to zero, then the target probabilities p_k
  // (spec_decode.py:48).
  double cexcl, total;
  double cincl = block_scan_f64(wv, shs1, cexcl, total);
  const int use_p = (dec.mode == kModeResidual && !(total > 0.0)) ? 1 : 0;  // uniform
  const double mass = use_p ? pv : wv;
  if (use_p) cincl = block_scan_f64(pv, shs2, cexcl, total);
  csum[tid] = cincl;
  const double tau = static_cast<double>(ures) * total;
  // the prefix is non-decreasing, so at most one chunk has excl <= tau < incl
  const bool has = tid < a.L.nch2 && mass > 0.0;
  const uint64_t cross = __ballot(has && cexcl <= tau && tau < cincl);
  const uint64_t hasm = __ballot(has);
  if (lane == 0) {
    sh_cross[wave] = cross ? wave * 64 + __builtin_ctzll(cross) : -1;
    sh_lastm[wave] = hasm ? wave * 64 + 63 - __builtin_clzll(hasm) : 0;
  }
  __syncthreads();
  // tau within rounding of the total: the last chunk with mass
  int chunk = -1, lastm = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (chunk < 0 && sh_cross[q] >= 0) chunk = sh_cross[q];
    lastm = max(lastm, sh_lastm[q]);
  }
  if (chunk < 0) chunk = lastm;
  const double acc = chunk == 0 ? 0.0 : csum[chunk - 1];
  const int clo = chunk * a.L.chunk2;
  const int chi = min(a.V, clo + a.L.chunk2);
  // each thread owns a contiguous run of 8-element groups of the chunk
  const int groups = (chi - clo + 7) / 8;
  const int per = (groups + kThreads - 1) / kThreads;
  const int tlo = min(chi, clo + tid * per * 8);
  const int thi = min(chi, tlo + per * 8);
  const bool vec = a.vec_t && (dec.mode == kModeBonus || a.vec_d);
  // The first kKeep groups of the thread's run stay in registers for the claim pass below.
  constexpr int kKeep = 4;
  float keep[kKeep][8];
  double local = 0.0;
  if (vec && ((thi - tlo) & 7) == 0 && chi - clo >= 8) {
    // every group of the run is full: all kKeep groups' loads first (groups past the run
    // reload the chunk's first group, in bounds and never used), then the same sums
    typename WeightRow<BF16>::Raw r[kKeep];
#pragma unroll
    for (int gi = 0; gi < kKeep; ++gi) {
      const int j = tlo + gi * 8;
      wr.load(j < thi ? j : clo, r[gi]);
    }
#pragma unroll
    for (int gi = 0; gi < kKeep; ++gi) {
#pragma unroll
      for (int e = 0; e < 8; ++e) keep[gi][e] = 0.0f;
      if (tlo + gi * 8 < thi) {
        float w[8], p[8];
        wr.finish(r[gi], w, p);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          keep[gi][e] = use_p ? p[e] : w[e];
          local += static_cast<double>(keep[gi][e]);
        }
      }
    }
  } else {
#pragma unroll
    for (int gi = 0; gi < kKeep; ++gi) {
      const int j = tlo + gi * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) keep[gi][e] = 0.0f;
      if (j < thi) {
        float w[8], p[8];
        const int n = min(8, thi - j);
        wr.at(j, n, vec && n == 8, w, p);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          keep[gi][e] = e < n ? (use_p ? p[e] : w[e]) : 0.0f;
          local += static_cast<double>(keep[gi][e]);
        }
      }
    }
  }
  for (int j = tlo + kKeep * 8; j < thi; j += 8) {
    float w[8], p[8];
    const int n = min(8, thi - j);
    wr.at(j, n, vec && n == 8, w, p);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n) local += static_cast<double>(use_p ? p[e] : w[e]);
  }
  double start, tot_unused;
  const double incl = block_scan_f64(local, shs3, start, tot_unused);
  // Thread t owns [acc + incl_{t-1}, acc + incl_t).
  const bool claim = (acc + start <= tau) && (tau < acc + incl) && (thi > tlo);
  int tok = -1;
  float mg = 0.0f;
  if (claim) {
    double run = acc + start;
    int last_pos = -1;
    double lo_edge = run, hi_edge = run;
    for (int j = tlo, gi = 0; j < thi && tok < 0; j += 8, ++gi) {
      float v[8];
      const int n = min(8, thi - j);
      if (gi < kKeep) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = keep[gi < kKeep ? gi : 0][e];
      } else {
        float w[8], p[8];
        wr.at(j, n, vec && n == 8, w, p);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = use_p ? p[e] : w[e];
      }
      for (int e = 0; e < n; ++e) {
        const double wj = static_cast<double>(v[e]);
        if (wj > 0.0) last_pos = j + e;
        const double nxt = run + wj;
        if (nxt > tau && wj > 0.0) {
          tok = j + e;
          lo_edge = run;
          hi_edge = nxt;
          break;
        }
        run = nxt;
      }
    }
    if (tok < 0) {
      tok = last_pos >= 0 ? last_pos : tlo;
    } else {
      mg = static_cast<float>(fmin(tau - lo_edge, hi_edge - tau) / total);
    }
    // fp64 rounding could in principle let two neighbours claim; the smaller index wins
    // (claimants own disjoint ranges, so their tokens differ).
    atomicMin(&sh_tok_min, tok);
  }
  __syncthreads();
  if (claim && tok == sh_tok_min) sh_margin = mg;
  __syncthreads();
  if (tid == 0) {
    int pick = sh_tok_min == 0x7fffffff ? -1 : sh_tok_min;
    float pick_margin = sh_margin;
    if (pick < 0) {  // nobody claimed (rounding at the chunk end): last element with mass
      for (int j = chi - 1; j >= clo && pick < 0; --j) {
        float w[8], p[8];
        wr.at(j, 1, false, w, p);
        if ((use_p ? p[0] : w[0]) > 0.0f) pick = j;
      }
      if (pick < 0) pick = clo;
      pick_margin = 0.0f;
    }
    a.out_tok[static_cast<int64_t>(b) * (a.gmax + 1) + dec.k] = pick;
    if (a.margin) a.margin[b] = fminf(dec.margin, pick_margin);
  }
}

// softmax(x * inv_t) per row, written as fp32 probabilities: one 1024-thread block per row
// and three passes -- the max, the fp64 sum of exp, then the write -- the second and third
// finding the row (a few hundred KB) in L2.  Rows aligned for it (vec_ok) are read in
// 8-element vector loads, kSmU groups in flight per thread; a group past the vector part
// re-reads the last one, and in the write pass stores the same bytes again, so no load sits
// under a branch.  (One 256-thread block with one 4-byte load per thread and step took
// ~250 us for 32 rows of 128256.)
constexpr int kSmThreads = 1024;
constexpr int kSmU = 4;

template <bool BF16>
__global__ __launch_bounds__(kSmThreads) void softmax_kernel(const void* x, int64_t in_stride, int V,
                                                             float inv_t, float* out,
                                                             int64_t out_stride, int vec_ok) {
  constexpr int kW = kSmThreads / 64;
  constexpr int kStep = kSmThreads * 8;
  __shared__ float shf[kW];
  __shared__ double shd[kW];
  const int64_t r = blockIdx.x;
  const int tid = static_cast<int>(threadIdx.x);
  const int V8 = vec_ok ? V / 8 * 8 : 0;
  float* orow = out + r * out_stride;
  float v[kSmU][8];
  auto load_round = [&](int j0) {
#pragma unroll
    for (int u = 0; u < kSmU; ++u) ld8<BF16>(x, r, in_stride, min(j0 + u * kStep, V8 - 8), v[u]);
  };
  // pass 1: the row max of x * inv_t
  float m = -INFINITY;
  for (int j0 = tid * 8; j0 < V8; j0 += kStep * kSmU) {
    load_round(j0);
#pragma unroll
    for (int u = 0; u < kSmU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) m = fmaxf(m, v[u][e] * inv_t);  // repeats change no max
  }
  for (int j = V8 + tid; j < V; j += kSmThreads) m = fmaxf(m, ld<BF16>(x, r, in_stride, j) * inv_t);
  m = wave_max_f32(m);
  if ((tid & 63) == 0) shf[tid >> 6] = m;
  __syncthreads();
  m = shf[0];
#pragma unroll
  for (int w = 1; w < kW; ++w) m = fmaxf(m, shf[w]);
  const float m_l2 = m * kLog2e;
  // pass 2: sum of exp(x * inv_t - m) in fp64
  double s = 0.0;
  for (int j0 = tid * 8; j0 < V8; j0 += kStep * kSmU) {
    load_round(j0);
#pragma unroll
    for (int u = 0; u < kSmU; ++u) {
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += exp_shift(v[u][e] * inv_t, m_l2);
      s += j0 + u * kStep < V8 ? static_cast<double>(acc) : 0.0;
    }
  }
  for (int j = V8 + tid; j < V; j += kSmThreads)
    s += static_cast<double>(exp_shift(ld<BF16>(x, r, in_stride, j) * inv_t, m_l2));
  s = wave_sum_f64(s);
  if ((tid & 63) == 0) shd[tid >> 6] = s;
  __syncthreads();
  s = 0.0;
#pragma unroll
  for (int w = 0; w < kW; ++w) s += shd[w];
  const double inv_s = 1.0 / s;
  // pass 3: the probabilities
  for (int j0 = tid * 8; j0 < V8; j0 += kStep * kSmU) {
    load_round(j0);
#pragma unroll
    for (int u = 0; u < kSmU; ++u) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        p[e] = static_cast<float>(static_cast<double>(exp_shift(v[u][e] * inv_t, m_l2)) * inv_s);
      float4* dst = reinterpret_cast<float4*>(orow + min(j0 + u * kStep, V8 - 8));
      dst[0] = make_float4(p[0], p[1], p[2], p[3]);
      dst[1] = make_float4(p[4], p[5], p[6], p[7]);
    }
  }
  for (int j = V8 + tid; j < V; j += kSmThreads) {
    const float xs = ld<BF16>(x, r, in_stride, j) * inv_t;
    orow[j] = static_cast<float>(static_cast<double>(exp_shift(xs, m_l2)) * inv_s);
  }
}

// Probabilities of a sampling call (gamma_max = 0) from the row statistics its row_stats
// launch left in the workspace: grid (element chunk, row).  A block issues its logit loads,
// then one wave combines the row's chunk partials into (M, S) (max, then sum of
// s_c exp(m_c - M), fp64), and every element becomes fp32(exp(x/T - M) / S) by the softmax
// kernel's formula.  Each element is read once and written once, by a grid that fills the GPU.
constexpr int kPrThreads = 256;
constexpr int kPrGroups = 2;  // 8-element groups per thread
constexpr int kPrChunk = kPrThreads * 8 * kPrGroups;

template <bool BF16>
__global__ __launch_bounds__(kPrThreads) void sample_probs_kernel(Args a, float* out,
                                                                  int64_t out_stride, int vec_ok) {
  __shared__ float sh_m;
  __shared__ double sh_inv;
  const int64_t r = blockIdx.y;
  const int tid = static_cast<int>(threadIdx.x);
  const int lo = static_cast<int>(blockIdx.x) * kPrChunk;
  const int V8 = vec_ok ? a.V / 8 * 8 : 0;
  float v[kPrGroups][8];
  if (V8 > 0) {
#pragma unroll
    for (int g = 0; g < kPrGroups; ++g)
      ld8<BF16>(a.tgt, r, a.tgt_stride, min(lo + (g * kPrThreads + tid) * 8, V8 - 8), v[g]);
  }
  if (tid < 64) {  // wave 0: the row's (M, S), its partials read in one round
    constexpr int kPL = 4;  // partials per lane held in registers
    const Partial1* p = a.ws.part1 + r * a.L.nch1;
    const int n = a.L.nch1;
    Partial1 q[kPL];
#pragma unroll
    for (int k = 0; k < kPL; ++k) q[k] = p[min(tid + 64 * k, n - 1)];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPL; ++k) m = fmaxf(m, q[k].m);  // a repeated partial changes no max
    for (int c = tid + 64 * kPL; c < n; c += 64) m = fmaxf(m, p[c].m);
    m = wave_max_f32(m);
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < kPL; ++k)
      if (tid + 64 * k < n && q[k].s > 0.0) s += q[k].s * exp(static_cast<double>(q[k].m) - static_cast<double>(m));
    for (int c = tid + 64 * kPL; c < n; c += 64) {
      const Partial1 e = p[c];
      if (e.s > 0.0) s += e.s * exp(static_cast<double>(e.m) - static_cast<double>(m));
    }
    s = wave_sum_f64(s);
    if (tid == 0) {
      sh_m = m;
      sh_inv = 1.0 / s;
    }
  }
  __syncthreads();
  const float m_l2 = sh_m * kLog2e;
  const double inv_s = sh_inv;
  float* orow = out + r * out_stride;
  if (V8 > 0) {
#pragma unroll
    for (int g = 0; g < kPrGroups; ++g) {
      const int j = lo + (g * kPrThreads + tid) * 8;
      if (j >= V8) continue;  // the loads above were clamped, not skipped
      float pr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pr[e] = static_cast<float>(static_cast<double>(exp_shift(v[g][e] * a.inv_t, m_l2)) * inv_s);
      float4* dst = reinterpret_cast<float4*>(orow + j);
      dst[0] = make_float4(pr[0], pr[1], pr[2], pr[3]);
      dst[1] = make_float4(pr[4], pr[5], pr[6], pr[7]);
    }
  }
  // elements past the vector part (or every element of an unaligned row)
  const int t0 = max(lo, V8), t1 = min(lo + kPrChunk, a.V);
  for (int j = t0 + tid; j < t1; j += kPrThreads) {
    const float xs = ld<BF16>(a.tgt, r, a.tgt_stride, j) * a.inv_t;
    orow[j] = static_cast<float>(static_cast<double>(exp_shift(xs, m_l2)) * inv_s);
  }
}

// ---------------------------------------------------------------------------------------
// Launch 2 (sampling at gamma_max = 0: sample(), engine/spec_decode.py:12-17): the decision
// and the chunk sums come from launch 1's partials, so one launch finishes the draw.
// Per row, wave 0 combines the chunk partials into (M, S) and the chunk masses
// P_c = s_c exp(m_c - M) / S (fp64); their prefix locates the chunk c* where the cumulative
// probability crosses tau = u * sum(P_c).  Within c* the cumulative sum runs over the fp32
// probabilities p_j = fp32(exp(x_j/T - M) / S) themselves (the values PROBS writes, and
// select_kernel's weights), in fp64.  A chunk mass differs from the sum of its p_j by a few
// 1e-7 of the total, so a draw within that of a chunk edge may land one element away from
// the exact cumulative sum's -- inside the 1e-6 band such draws are reported in.
// Grid (chunk, row): block c issues the loads of chunk c (kDrawG groups of 8 elements a
// thread) before wave 0 combines the statistics, so no load waits on the decision; PROBS:
// every block writes its chunk's probabilities; the block of chunk c* then draws from the
// probabilities in its registers, and the other blocks are done.
// ---------------------------------------------------------------------------------------
constexpr int kPL = 8;  // chunk partials a lane of wave 0 keeps in registers

// (M, 1 / S) of row b from its chunk partials, and with DRAW the crossing chunk: wave 0 only.
// Rows of more than 64 * kPL chunks (vocabularies past 8M) read the rest again per pass.
struct RowDraw {
  float m;
  double inv, total, tau, acc;
  int chunk;
};
struct RowPartials {
  Partial1 q[kPL];
};
// Issues wave 0's loads of row b's first 64 * kPL chunk partials.
__device__ __forceinline__ void load_row_partials(const Args& a, int b, RowPartials& rp) {
  const int lane = threadIdx.x & 63;
  const Partial1* part = a.ws.part1 + static_cast<int64_t>(b) * a.L.nch1;
  const int n = a.L.nch1, nk = (n + 63) / 64;
  // unconditional loads of a clamped index keep the compiler's wait counts exact; chunks past
  // the row are masked where row_draw reads them (a mask here would wait for the loads)
  (void)nk;
#pragma unroll
  for (int k = 0; k < kPL; ++k) rp.q[k] = part[min(lane + 64 * k, n - 1)];
}
template <bool DRAW>
__device__ __forceinline__ RowDraw row_draw(const Args& a, int b, float u, const RowPartials& rp) {
  const int lane = threadIdx.x & 63;
  const Partial1* part = a.ws.part1 + static_cast<int64_t>(b) * a.L.nch1;
  const int n = a.L.nch1, nk = (n + 63) / 64;
  Partial1 q[kPL];
#pragma unroll
  for (int k = 0; k < kPL; ++k) {
    const bool in = k < nk && lane + 64 * k < n;
    q[k].m = in ? rp.q[k].m : -INFINITY;
    q[k].s = in ? rp.q[k].s : 0.0;
    q[k].idx = -1;
  }
  auto far = [&](int k) {  // partial of chunk lane + 64 k, k >= kPL
    return lane + 64 * k < n ? part[lane + 64 * k] : Partial1{-INFINITY, -1, 0.0};
  };
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPL; ++k) m = fmaxf(m, q[k].m);
  for (int k = kPL; k < nk; ++k) m = fmaxf(m, far(k).m);
  m = wave_max_f32_dpp(m);
  auto mass_of = [&](const Partial1& x) {
    return x.s > 0.0 ? x.s * exp(static_cast<double>(x.m) - static_cast<double>(m)) : 0.0;
  };
  double ms[kPL];
  double S = 0.0;
#pragma unroll
  for (int k = 0; k < kPL; ++k) {
    ms[k] = 0.0;
    if (k < nk) {  // uniform
      ms[k] = mass_of(q[k]);
      S += ms[k];
    }
  }
  for (int k = kPL; k < nk; ++k) S += mass_of(far(k));
  S = wave_sum_f64_dpp(S);
  RowDraw r{};
  r.m = m;
  r.inv = 1.0 / S;
  if constexpr (DRAW) {
    const double inv = r.inv;
    double total = 0.0;
#pragma unroll
    for (int k = 0; k < kPL; ++k)
      if (k < nk) total += ms[k] * inv;
    for (int k = kPL; k < nk; ++k) total += mass_of(far(k)) * inv;
    total = wave_sum_f64_dpp(total);
    const double tau = static_cast<double>(u) * total;
    // the first chunk with mass whose [prefix, prefix + P_c) holds tau; tau within rounding
    // of the total: the last chunk with mass
    double run = 0.0, acc = 0.0, acc_last = 0.0;
    int chunk = -1, lastm = 0;
    auto scan64 = [&](int k, double pc) {  // chunks 64 k .. 64 k + 63, this lane's mass pc
      double ex;
      const double in = wave_incl_scan_f64(pc, ex) + run;
      ex = lane == 0 ? run : ex + run;
      const uint64_t cr = __ballot(pc > 0.0 && ex <= tau && tau < in);
      const uint64_t hm = __ballot(pc > 0.0);
      if (chunk < 0 && cr) {
        const int l = __builtin_ctzll(cr);
        chunk = 64 * k + l;
        acc = __shfl(ex, l, 64);
      }
      if (hm) {
        const int l = 63 - __builtin_clzll(hm);
        lastm = 64 * k + l;
        acc_last = __shfl(ex, l, 64);
      }
      run = __shfl(in, 63, 64);
    };
#pragma unroll
    for (int k = 0; k < kPL; ++k)
      if (k < nk) scan64(k, ms[k] * inv);
    for (int k = kPL; k < nk; ++k) scan64(k, mass_of(far(k)) * inv);
    if (chunk < 0) {
      chunk = lastm;
      acc = acc_last;
    }
    r.total = total;
    r.tau = tau;
    r.acc = acc;
    r.chunk = chunk;
  }
  return r;
}

template <bool BF16, bool PROBS>
__global__ __launch_bounds__(kThreads) void sample_select_kernel(Args a, float* probs,
                                                                 int64_t probs_stride, int vec_out) {
  constexpr int kG = kDrawG;  // 8-element groups per thread
  __shared__ float sh_m;
  __shared__ double sh_inv, sh_total, sh_tau, sh_acc;
  __shared__ int sh_chunk;
  __shared__ double sh_pass[4][kG];
  __shared__ double sh_scan[4];
  __shared__ int sh_tok, sh_last;
  __shared__ float sh_mg;
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = tgt_row(a, b, 0);
  const float ures = a.u_res[b];
  const int lo = c * a.L.chunk1, hi = min(a.V, lo + a.L.chunk1);
  // group (it, t) covers elements lo + (it * kThreads + t) * 8 ..: pass it is the contiguous
  // range [lo + it * kThreads * 8, +kThreads * 8) in thread order
  float vals[kG * 8];
  // a full chunk of aligned rows (readfirstlane: the compiler then knows the branch is
  // uniform and keeps the two load paths apart, so no load waits for the other path's)
  const bool full = __builtin_amdgcn_readfirstlane(a.vec_t && hi - lo == a.L.chunk1 ? 1 : 0) != 0;
  if (full) {  // out-of-chunk groups re-load the chunk's first group (masked below)
#pragma unroll
    for (int it = 0; it < kG; ++it) {
      const int j0 = lo + (it * kThreads + tid) * 8;
      ld8<BF16>(a.tgt, row, a.tgt_stride, j0 < hi ? j0 : lo, vals + it * 8);
    }
  } else {
#pragma unroll
    for (int it = 0; it < kG; ++it)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = lo + (it * kThreads + tid) * 8 + e;
        vals[it * 8 + e] = j < hi ? ld<BF16>(a.tgt, row, a.tgt_stride, j) : -INFINITY;
      }
  }
  // the partials' loads go out right behind the chunk's (all in flight together)
  RowPartials rp;
  if (wave == 0) load_row_partials(a, b, rp);
  if (tid == 0) {
    sh_tok = 0x7fffffff;
    sh_last = -1;
    sh_mg = 0.0f;
  }
  if (wave == 0) {
    const RowDraw r = row_draw<true>(a, b, ures, rp);
    if (lane == 0) {
      sh_m = r.m;
      sh_inv = r.inv;
      sh_total = r.total;
      sh_tau = r.tau;
      sh_acc = r.acc;
      sh_chunk = r.chunk;
    }
  }
  __syncthreads();
  const bool draws = c == sh_chunk;  // uniform
  if (!PROBS && !draws) return;
  const float m_l2 = sh_m * kLog2e;
  const double inv = sh_inv;
  float* const pv = vals;  // the probabilities replace the logits in place
#pragma unroll
  for (int it = 0; it < kG; ++it)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = lo + (it * kThreads + tid) * 8 + e;
      const float x = j < hi ? vals[it * 8 + e] : -INFINITY;
      pv[it * 8 + e] = static_cast<float>(static_cast<double>(exp_shift(x * a.inv_t, m_l2)) * inv);
    }
  if constexpr (PROBS) {
    float* orow = probs + static_cast<int64_t>(b) * probs_stride;
#pragma unroll
    for (int it = 0; it < kG; ++it) {
      const int j0 = lo + (it * kThreads + tid) * 8;
      const float* q = pv + it * 8;
      if (vec_out && full) {
        if (j0 < hi) {
          float4* dst = reinterpret_cast<float4*>(orow + j0);
          dst[0] = make_float4(q[0], q[1], q[2], q[3]);
          dst[1] = make_float4(q[4], q[5], q[6], q[7]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (j0 + e < hi) orow[j0 + e] = q[e];
      }
    }
    if (!draws) return;
  }
  // ---- the draw, in chunk c* ----
  double gs[kG];
  int last = -1;  // the last element with mass (fallback when tau lies past the element sum)
#pragma unroll
  for (int it = 0; it < kG; ++it) {
    double d8 = 0.0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      d8 += static_cast<double>(pv[it * 8 + e]);
      if (pv[it * 8 + e] > 0.0f) last = lo + (it * kThreads + tid) * 8 + e;
    }
    gs[it] = d8;
    const double w = wave_sum_f64_dpp(d8);
    if (lane == 0) sh_pass[wave][it] = w;
  }
  atomicMax(&sh_last, last);
  __syncthreads();
  const double tau = sh_tau, total = sh_total;
  double run = sh_acc;
  int pass = -1;
  double pass_acc = 0.0;
#pragma unroll
  for (int it = 0; it < kG; ++it) {
    const double T = ((sh_pass[0][it] + sh_pass[1][it]) + sh_pass[2][it]) + sh_pass[3][it];
    if (pass < 0 && T > 0.0 && run <= tau && tau < run + T) {
      pass = it;
      pass_acc = run;
    }
    run += T;
  }
  bool claim = false;
  int tok = -1;
  float mg = 0.0f;
  if (pass >= 0) {  // uniform
    double g = 0.0;
#pragma unroll
    for (int it = 0; it < kG; ++it) g = it == pass ? gs[it] : g;
    double excl, tot_unused;
    const double incl = block_scan_f64(g, sh_scan, excl, tot_unused);
    claim = g > 0.0 && pass_acc + excl <= tau && tau < pass_acc + incl;
    if (claim) {
      float w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = 0.0f;
#pragma unroll
        for (int it = 0; it < kG; ++it) x = it == pass ? pv[it * 8 + e] : x;
        w[e] = x;
      }
      const int j0 = lo + (pass * kThreads + tid) * 8;
      double r = pass_acc + excl;
      int lastw = -1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double wj = static_cast<double>(w[e]);
        const double nxt = r + wj;
        if (tok < 0) {
          if (wj > 0.0) lastw = j0 + e;
          if (nxt > tau && wj > 0.0) {
            tok = j0 + e;
            mg = static_cast<float>(fmin(tau - r, nxt - tau) / total);
          }
          r = nxt;
        }
      }
      if (tok < 0) tok = lastw;  // rounding inside the group: its last element with mass
      atomicMin(&sh_tok, tok);
    }
  }
  __syncthreads();
  if (claim && tok == sh_tok) sh_mg = mg;
  __syncthreads();
  if (tid == 0) {
    int pick = sh_tok == 0x7fffffff ? -1 : sh_tok;
    float pm = sh_mg;
    if (pick < 0) {  // nobody claimed (tau past the chunk's element sum): its last element with mass
      pick = sh_last >= 0 ? sh_last : lo;
      pm = 0.0f;
    }
    a.out_tok[static_cast<int64_t>(b) * (a.gmax + 1)] = pick;
    if (a.acc_len) a.acc_len[b] = 0;  // null for coopt_sample (tokens only)
    if (a.margin) a.margin[b] = pm;
  }
}

// probs: gamma_max = 0 only -- the softmax rows written by the draw's second launch.
template <bool BF16>
int launch_all(Args& a, bool greedy, hipStream_t s, float* probs = nullptr,
               int64_t probs_stride = 0, int vec_out = 0) {
  const dim3 g1(a.L.nch1, 2 * a.gmax + 1, a.B);
  if (greedy)
    hipLaunchKernelGGL((row_stats_kernel<BF16, true>), g1, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((row_stats_kernel<BF16, false>), g1, dim3(kThreads), 0, s, a);
  int rc = coopt::check_launch("coopt_accept_sample/row_stats");
  if (rc != COOPT_OK) return rc;
  if (greedy) {
    hipLaunchKernelGGL(greedy_kernel, dim3(a.B), dim3(kThreads), 0, s, a);
    return coopt::check_launch("coopt_accept_sample/greedy");
  }
  if (a.gmax == 0) {  // a plain draw: the decision and chunk sums follow from the partials
    const dim3 grid(a.L.nch1, a.B);
    if (probs)
      hipLaunchKernelGGL((sample_select_kernel<BF16, true>), grid, dim3(kThreads), 0, s, a, probs,
                         probs_stride, vec_out);
    else
      hipLaunchKernelGGL((sample_select_kernel<BF16, false>), grid, dim3(kThreads), 0, s, a,
                         nullptr, 0, 0);
    return coopt::check_launch("coopt_accept_sample/sample_select");
  }
  // rows of at most 16 chunk partials are combined by lane groups, one partial per thread
  const dim3 g2(a.L.nch2, a.B);
  if (a.L.nch1 <= 8)
    hipLaunchKernelGGL((decide_kernel<BF16, 8>), g2, dim3(kThreads), 0, s, a);
  else if (a.L.nch1 <= 16)
    hipLaunchKernelGGL((decide_kernel<BF16, 16>), g2, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((decide_kernel<BF16, 0>), g2, dim3(kThreads), 0, s, a);
  rc = coopt::check_launch("coopt_accept_sample/decide");
  if (rc != COOPT_OK) return rc;
  hipLaunchKernelGGL((select_kernel<BF16>), dim3(a.B), dim3(kThreads), 0, s, a);
  return coopt::check_launch("coopt_accept_sample/select");
}

}  // namespace

extern "C" size_t coopt_accept_sample_workspace(int B, int gamma_max, int V) {
  if (B <= 0 || gamma_max < 0 || V <= 0) return 0;
  const Layout L = make_layout(B, gamma_max, V);
  Workspace w;
  return carve(&w, 0, B, gamma_max, L);
}

extern "C" int coopt_accept_sample(int logits_dtype, const void* target, int64_t target_row_stride,
                                   const int32_t* target_row0, int draft_kind, const void* draft,
                                   int64_t draft_row_stride, const int32_t* draft_row0,
                                   const int32_t* draft_tokens, const int32_t* gamma_per_seq,
                                   const float* u_accept, const float* u_resample,
                                   float temperature, int B, int gamma_max, int V,
                                   int32_t* accepted_len, int32_t* out_tokens, float* margin,
                                   void* workspace, size_t workspace_bytes,
                                   coopt_stream_t stream) {
  COOPT_REQUIRE(logits_dtype == COOPT_DT_F32 || logits_dtype == COOPT_DT_BF16,
                "logits_dtype must be F32 or BF16");
  COOPT_REQUIRE(B >= 0 && gamma_max >= 0 && gamma_max <= 64 && V > 0, "bad sizes");
  COOPT_REQUIRE(B <= 65535, "B must be <= 65535");
  if (B == 0) return COOPT_OK;
  const bool greedy = !(temperature > 0.0f);
  COOPT_REQUIRE(target && accepted_len && out_tokens && workspace, "null pointer");
  COOPT_REQUIRE(target_row_stride >= V, "target_row_stride < V");
  if (gamma_max > 0) COOPT_REQUIRE(draft_tokens != nullptr, "draft_tokens is null");
  if (!greedy) {
    COOPT_REQUIRE(u_resample != nullptr, "u_resample is null");
    if (gamma_max > 0) {
      COOPT_REQUIRE(draft && u_accept, "draft / u_accept is null");
      COOPT_REQUIRE(draft_kind == 0 || draft_kind == 1, "draft_kind must be 0 (logits) or 1 (probs)");
      COOPT_REQUIRE(draft_row_stride >= V, "draft_row_stride < V");
    }
  }
  const size_t need = coopt_accept_sample_workspace(B, gamma_max, V);
  if (workspace_bytes < need) {
    coopt::set_error("coopt_accept_sample: workspace too small");
    return COOPT_EWORKSPACE;
  }
  coopt::clear_error();
  const bool bf16 = logits_dtype == COOPT_DT_BF16;
  Args a{};
  a.tgt = target;
  a.tgt_stride = target_row_stride;
  a.tgt_row0 = target_row0;
  a.drf = draft;
  a.drf_stride = draft_row_stride;
  a.drf_row0 = draft_row0;
  a.dtok = draft_tokens;
  a.gam = gamma_per_seq;
  a.u_acc = u_accept;
  a.u_res = u_resample;
  a.acc_len = accepted_len;
  a.out_tok = out_tokens;
  a.margin = margin;
  // torch's GPU path evaluates "logits / T" as logits * fp32(1/T).
  a.inv_t = greedy ? 1.0f : 1.0f / temperature;
  a.draft_probs = (draft_kind == 1) ? 1 : 0;
  // 16-byte loads need 16-byte aligned rows (stride a multiple of 8 bf16 / 4 fp32 elements).
  a.vec_t = coopt::aligned16(target) && target_row_stride % (bf16 ? 8 : 4) == 0;
  const int dq = (bf16 && draft_kind == 0) ? 8 : 4;
  a.vec_d = draft != nullptr && coopt::aligned16(draft) && draft_row_stride % dq == 0;
  a.B = B;
  a.gmax = gamma_max;
  a.V = V;
  a.L = make_layout(B, gamma_max, V);
  carve(&a.ws, reinterpret_cast<uintptr_t>(workspace), B, gamma_max, a.L);
  auto s = static_cast<hipStream_t>(stream);
  return bf16 ? launch_all<true>(a, greedy, s) : launch_all<false>(a, greedy, s);
}

// ---- the entry point that allocates nothing ----------------------------------------------
// Its workspace is this file-scope device array: each GPU the library runs on holds its own
// copy (kAcceptScratchBytes) until the process ends.  Host code never passes the array's name
// to a kernel -- on the host that name is a stand-in, not a device address -- but the address
// hipGetSymbolAddress returns for the current device, looked up once per device.
namespace {

constexpr size_t kAcceptScratchBytes = size_t{2} << 20;
__device__ __align__(256) unsigned char scratch[kAcceptScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (nullptr with the error recorded on failure).
void* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    coopt::set_error("coopt_accept_sample_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || p == nullptr) {
      coopt::set_error(std::string("coopt_accept_sample_noalloc: hipGetSymbolAddress: ") +
                       hipGetErrorString(rc));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" size_t coopt_accept_sample_noalloc_max_bytes(void) { return kAcceptScratchBytes; }

extern "C" int coopt_accept_sample_noalloc(int logits_dtype, const void* target,
                                           int64_t target_row_stride, const int32_t* target_row0,
                                           int draft_kind, const void* draft,
                                           int64_t draft_row_stride, const int32_t* draft_row0,
                                           const int32_t* draft_tokens,
                                           const int32_t* gamma_per_seq, const float* u_accept,
                                           const float* u_resample, float temperature, int B,
                                           int gamma_max, int V, int32_t* accepted_len,
                                           int32_t* out_tokens, float* margin,
                                           coopt_stream_t stream) {
  COOPT_REQUIRE(B >= 0 && gamma_max >= 0 && gamma_max <= 64 && V > 0, "bad sizes");
  if (B == 0) return COOPT_OK;
  const size_t need = coopt_accept_sample_workspace(B, gamma_max, V);
  if (need > kAcceptScratchBytes) {
    coopt::set_error("coopt_accept_sample_noalloc: B=" + std::to_string(B) + ", gamma_max=" +
                     std::to_string(gamma_max) + ", V=" + std::to_string(V) + " need " +
                     std::to_string(need) + " bytes of scratch, more than its " +
                     std::to_string(kAcceptScratchBytes) + "; use coopt_accept_sample with a "
                     "caller workspace");
    return COOPT_EWORKSPACE;
  }
  void* ws = scratch_ptr();
  if (ws == nullptr) return COOPT_EHIP;
  return coopt_accept_sample(logits_dtype, target, target_row_stride, target_row0, draft_kind,
                             draft, draft_row_stride, draft_row0, draft_tokens, gamma_per_seq,
                             u_accept, u_resample, temperature, B, gamma_max, V, accepted_len,
                             out_tokens, margin, ws, kAcceptScratchBytes, stream);
}

extern "C" int coopt_softmax(int logits_dtype, const void* logits, int64_t in_stride, int64_t rows,
                             int V, float temperature, float* probs, int64_t out_stride,
                             coopt_stream_t stream) {
  COOPT_REQUIRE(logits_dtype == COOPT_DT_F32 || logits_dtype == COOPT_DT_BF16,
                "logits_dtype must be F32 or BF16");
  COOPT_REQUIRE(rows >= 0 && V > 0 && in_stride >= V && out_stride >= V, "bad sizes");
  COOPT_REQUIRE(temperature > 0.0f, "temperature must be > 0");
  if (rows == 0) return COOPT_OK;
  COOPT_REQUIRE(logits && probs, "null pointer");
  coopt::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  const float inv_t = 1.0f / temperature;
  const bool bf16 = logits_dtype == COOPT_DT_BF16;
  const int vec_ok = V >= 8 && (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 &&
                     in_stride % (bf16 ? 8 : 4) == 0 && (reinterpret_cast<uintptr_t>(probs) & 15u) == 0 &&
                     out_stride % 4 == 0;
  if (bf16)
    hipLaunchKernelGGL(softmax_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(kSmThreads), 0, s,
                       logits, in_stride, V, inv_t, probs, out_stride, vec_ok);
  else
    hipLaunchKernelGGL(softmax_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(kSmThreads), 0, s,
                       logits, in_stride, V, inv_t, probs, out_stride, vec_ok);
  return coopt::check_launch("coopt_softmax");
}

extern "C" int coopt_sample(int logits_dtype, const void* logits, int64_t row_stride, int N, int V,
                            float temperature, const float* uniforms, int32_t* tokens,
                            float* margin, float* probs, int64_t probs_stride, void* workspace,
                            size_t workspace_bytes, coopt_stream_t stream) {
  COOPT_REQUIRE(logits_dtype == COOPT_DT_F32 || logits_dtype == COOPT_DT_BF16,
                "logits_dtype must be F32 or BF16");
  COOPT_REQUIRE(N >= 0 && N <= 65535 && V > 0 && row_stride >= V, "bad sizes");
  COOPT_REQUIRE(temperature > 0.0f, "temperature must be > 0 (greedy rows: coopt_accept_sample)");
  COOPT_REQUIRE(!probs || probs_stride >= V, "probs_stride < V");
  if (N == 0) return COOPT_OK;
  COOPT_REQUIRE(logits && uniforms && tokens && workspace, "null pointer");
  const size_t need = coopt_accept_sample_workspace(N, 0, V);
  if (workspace_bytes < need) {
    coopt::set_error("coopt_sample: workspace too small");
    return COOPT_EWORKSPACE;
  }
  coopt::clear_error();
  const bool bf16 = logits_dtype == COOPT_DT_BF16;
  Args a{};
  a.tgt = logits;
  a.tgt_stride = row_stride;
  a.u_res = uniforms;
  a.out_tok = tokens;
  a.margin = margin;
  a.inv_t = 1.0f / temperature;
  a.vec_t = coopt::aligned16(logits) && row_stride % (bf16 ? 8 : 4) == 0;
  a.B = N;
  a.gmax = 0;
  a.V = V;
  a.L = make_layout(N, 0, V);
  carve(&a.ws, reinterpret_cast<uintptr_t>(workspace), N, 0, a.L);
  const int vec_out = probs != nullptr && coopt::aligned16(probs) && probs_stride % 4 == 0;
  auto s = static_cast<hipStream_t>(stream);
  return bf16 ? launch_all<true>(a, false, s, probs, probs_stride, vec_out)
              : launch_all<false>(a, false, s, probs, probs_stride, vec_out);
}

extern "C" int coopt_sample_probs(int logits_dtype, const void* logits, int64_t in_stride, int B,
                                  int V, float temperature, const void* workspace,
                                  size_t workspace_bytes, float* probs, int64_t out_stride,
                                  coopt_stream_t stream) {
  COOPT_REQUIRE(logits_dtype == COOPT_DT_F32 || logits_dtype == COOPT_DT_BF16,
                "logits_dtype must be F32 or BF16");
  COOPT_REQUIRE(B >= 0 && B <= 65535 && V > 0 && in_stride >= V && out_stride >= V, "bad sizes");
  COOPT_REQUIRE(temperature > 0.0f, "temperature must be > 0");
  if (B == 0) return COOPT_OK;
  COOPT_REQUIRE(logits && probs && workspace, "null pointer");
  const size_t need = coopt_accept_sample_workspace(B, 0, V);
  if (workspace_bytes < need) {
    coopt::set_error("coopt_sample_probs: workspace too small");
    return COOPT_EWORKSPACE;
  }
  coopt::clear_error();
  const bool bf16 = logits_dtype == COOPT_DT_BF16;
  Args a{};
  a.tgt = logits;
  a.tgt_stride = in_stride;
  a.inv_t = 1.0f / temperature;
  a.B = B;
  a.gmax = 0;
  a.V = V;
  a.L = make_layout(B, 0, V);
  carve(&a.ws, reinterpret_cast<uintptr_t>(const_cast<void*>(workspace)), B, 0, a.L);
  const int vec_ok = V >= 8 && coopt::aligned16(logits) && in_stride % (bf16 ? 8 : 4) == 0 &&
                     coopt::aligned16(probs) && out_stride % 4 == 0;
  const dim3 grid(static_cast<unsigned>((V + kPrChunk - 1) / kPrChunk), static_cast<unsigned>(B));
  auto s = static_cast<hipStream_t>(stream);
  if (bf16)
    hipLaunchKernelGGL(sample_probs_kernel<true>, grid, dim3(kPrThreads), 0, s, a, probs, out_stride, vec_ok);
  else
    hipLaunchKernelGGL(sample_probs_kernel<false>, grid, dim3(kPrThreads), 0, s, a, probs, out_stride, vec_ok);
  return coopt::check_launch("coopt_sample_probs");
}
