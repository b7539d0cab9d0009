// Fused speculative acceptance: vocab-wide softmax of target and draft rows, the p/q accept
// test, first rejection, the max(0, p - q) residual and inverse-CDF resampling, for a whole
// batch in two launches.  Semantics: engine/spec_decode.py:20-49 (sampling) and :30-35
// (greedy), looped over the batch at engine/engine.py:421-446, with the uniforms explicit.
//
// Launch 1 (row_stats_kernel), grid (chunk, row slot, sequence): every block reduces one
// chunk of one row -- max and an fp64 sum of exp(x/T - max) (sampling), or max and first
// argmax (greedy).  The last block to finish for a sequence (device-scope counter) combines
// the chunk partials into row statistics and runs the accept loop, which needs only the
// logits at the draft tokens; it writes the accepted prefix and the decision (k, which
// distribution to resample from).
// Launch 2 (resample_kernel), grid (chunk, sequence): partial fp64 sums of the resampling
// weights w_j; the last block of a sequence locates the chunk where the cumulative weight
// crosses u * sum(w), scans that chunk and writes the emitted token.
//
// Numerics.  Row maxima are exact; sum(exp) is accumulated in fp64 from fp32 expf terms; the
// probabilities at the draft tokens are formed in fp64 and rounded once to fp32, so p_i[d_i]
// and q_i[d_i] agree with an exactly rounded fp32 softmax except within an ulp of a rounding
// boundary.  Cumulative weights are fp64 sums of fp32 w_j.
#include <math.h>

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 64;                  // elements a phase-1 thread keeps in VGPRs
constexpr int kMaxChunk = kThreads * kMaxPerThread;  // 16384
constexpr int kMinChunk = 1024;

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
// without the data.
__host__ __device__ inline Layout make_layout(int B, int gmax, int V) {
  Layout L;
  const int rows = B * (2 * gmax + 1);
  int nch = ceil_div(2048, rows > 0 ? rows : 1);
  nch = imax(nch, ceil_div(V, kMaxChunk));
  nch = imin(nch, imax(1, ceil_div(V, kMinChunk)));
  L.chunk1 = ceil_div(ceil_div(V, nch), 8) * 8;
  L.nch1 = ceil_div(V, L.chunk1);
  int nch2 = ceil_div(1024, B > 0 ? B : 1);
  nch2 = imax(1, imin(nch2, ceil_div(V, kMinChunk)));
  L.chunk2 = ceil_div(ceil_div(V, nch2), 8) * 8;
  L.nch2 = ceil_div(V, L.chunk2);
  return L;
}

struct Workspace {
  unsigned* cnt1;    // [B]
  unsigned* cnt2;    // [B]
  Partial1* part1;   // [B][2*gmax+1][nch1]
  RowStat* rows;     // [B][2*gmax+1]
  Decision* dec;     // [B]
  Partial2* part2;   // [B][nch2]
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
  // two counters per sequence inside the fixed counter region (B <= kMaxCounters / 2)
  w->cnt1 = reinterpret_cast<unsigned*>(base);
  w->cnt2 = reinterpret_cast<unsigned*>(base + kCounterRegionBytes / 2);
  off = kCounterRegionBytes;
  w->part1 = reinterpret_cast<Partial1*>(take(sizeof(Partial1) * B * slots * L.nch1));
  w->rows = reinterpret_cast<RowStat*>(take(sizeof(RowStat) * B * slots));
  w->dec = reinterpret_cast<Decision*>(take(sizeof(Decision) * B));
  w->part2 = reinterpret_cast<Partial2*>(take(sizeof(Partial2) * B * L.nch2));
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
  int greedy;
  int draft_probs;
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

// Loads elements [lo, hi) of a row into vals[], thread-strided in groups of 4 (fp32) or 8
// (bf16) consecutive elements so that every wave instruction reads one contiguous span.
template <bool BF16>
__device__ __forceinline__ void load_chunk(const void* base, int64_t row, int64_t stride, int lo,
                                           int hi, bool vec_ok, float (&vals)[kMaxPerThread]) {
  constexpr int W = BF16 ? 8 : 4;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < kMaxPerThread / W; ++it) {
    const int j0 = lo + (it * kThreads + tid) * W;
    if (vec_ok && j0 + W <= hi) {
      if constexpr (BF16) {
        const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + row * stride + j0);
        const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) vals[it * W + e] = bf16_to_f32(static_cast<uint16_t>(w4[e / 2] >> (16 * (e & 1))));
      } else {
        const float4 r = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + row * stride + j0);
        vals[it * W + 0] = r.x;
        vals[it * W + 1] = r.y;
        vals[it * W + 2] = r.z;
        vals[it * W + 3] = r.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const int j = j0 + e;
        vals[it * W + e] = j < hi ? ld<BF16>(base, row, stride, j) : -INFINITY;
      }
    }
  }
}

// Block-wide reductions over kThreads threads (4 waves) through LDS.
__device__ __forceinline__ float block_max(float v, float* sh) {
  v = wave_max_f32(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum(double v, double* sh) {
  v = wave_sum_f64(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  double r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
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

// Accurate p = exp(x' - m) / s rounded once to fp32 (x' = fl32(x * inv_t)).
__device__ __forceinline__ float prob_at(float xs, float m, double s) {
  return static_cast<float>(exp(static_cast<double>(xs) - static_cast<double>(m)) / s);
}

template <bool BF16>
__device__ void finalize_sequence(const Args& a, int b) {
  const int g = gamma_of(a, b);
  const int slots = 2 * a.gmax + 1;
  const int nrow_t = g + 1;
  const int nrow_d = (a.greedy || a.draft_probs) ? 0 : g;
  const int tid = threadIdx.x;
  // Combine chunk partials into row statistics, one thread per row, in chunk order.
  if (tid < nrow_t + nrow_d) {
    const int slot = tid < nrow_t ? tid : (a.gmax + 1) + (tid - nrow_t);
    const Partial1* p = a.ws.part1 + (static_cast<int64_t>(b) * slots + slot) * a.L.nch1;
    RowStat rs;
    if (a.greedy) {
      float v = -INFINITY;
      int idx = 0x7fffffff;
      for (int c = 0; c < a.L.nch1; ++c) {
        const float pv = load_agent(&p[c].m);
        const int pi = load_agent(&p[c].idx);
        amax_merge(v, idx, pv, pi);
      }
      rs.m = v;
      rs.argmax = idx;
      rs.s = 0.0;
    } else {
      float m = -INFINITY;
      for (int c = 0; c < a.L.nch1; ++c) m = fmaxf(m, load_agent(&p[c].m));
      double s = 0.0;
      for (int c = 0; c < a.L.nch1; ++c) {
        const float pm = load_agent(&p[c].m);
        const double ps = load_agent(&p[c].s);
        if (ps > 0.0) s += ps * exp(static_cast<double>(pm) - static_cast<double>(m));
      }
      rs.m = m;
      rs.argmax = -1;
      rs.s = s;
    }
    a.ws.rows[static_cast<int64_t>(b) * slots + slot] = rs;
  }
  __syncthreads();
  __threadfence_block();
  if (tid != 0) return;

  const RowStat* rows = a.ws.rows + static_cast<int64_t>(b) * slots;
  const int32_t* d = a.dtok + static_cast<int64_t>(b) * a.gmax;
  int32_t* out = a.out_tok + static_cast<int64_t>(b) * (a.gmax + 1);
  int k = g;
  float margin = INFINITY;
  if (a.greedy) {
    for (int i = 0; i < g; ++i) {
      if (rows[i].argmax != d[i]) {
        k = i;
        break;
      }
    }
    for (int i = 0; i < k; ++i) out[i] = d[i];
    out[k] = rows[k].argmax;
    for (int i = k + 1; i <= a.gmax; ++i) out[i] = -1;
    a.acc_len[b] = k;
    if (a.margin) a.margin[b] = INFINITY;
    return;
  }
  const float* u = a.u_acc + static_cast<int64_t>(b) * a.gmax;
  int mode = kModeBonus;
  for (int i = 0; i < g; ++i) {
    const int tok = d[i];
    float ratio = 0.0f;
    if (tok >= 0 && tok < a.V) {
      const float xt = ld<BF16>(a.tgt, tgt_row(a, b, i), a.tgt_stride, tok) * a.inv_t;
      const float p = prob_at(xt, rows[i].m, rows[i].s);
      float q;
      if (a.draft_probs) {
        q = static_cast<const float*>(a.drf)[drf_row(a, b, i) * a.drf_stride + tok];
      } else {
        const float xq = ld<BF16>(a.drf, drf_row(a, b, i), a.drf_stride, tok) * a.inv_t;
        const RowStat& rq = rows[a.gmax + 1 + i];
        q = prob_at(xq, rq.m, rq.s);
      }
      ratio = fminf(p / fmaxf(q, 1e-20f), 1.0f);
    }
    margin = fminf(margin, fabsf(u[i] - ratio));
    if (u[i] >= ratio) {
      k = i;
      mode = kModeResidual;
      break;
    }
  }
  for (int i = 0; i < k; ++i) out[i] = d[i];
  for (int i = k + 1; i <= a.gmax; ++i) out[i] = -1;
  a.acc_len[b] = k;
  Decision dec;
  dec.k = k;
  dec.mode = mode;
  dec.margin = margin;
  dec.pad = 0;
  a.ws.dec[b] = dec;
}

template <bool BF16>
__global__ __launch_bounds__(kThreads) void row_stats_kernel(Args a) {
  __shared__ float shf[4];
  __shared__ double shd[4];
  __shared__ float shv[4];
  __shared__ int shi[4];
  __shared__ int last;
  const int c = blockIdx.x, slot = blockIdx.y, b = blockIdx.z;
  const int g = gamma_of(a, b);
  const bool is_draft = slot > a.gmax;
  const int i = is_draft ? slot - a.gmax - 1 : slot;
  if (!is_draft && i > g) return;
  if (is_draft && (a.greedy || a.draft_probs || i >= g)) return;

  const void* base = is_draft ? a.drf : a.tgt;
  const int64_t stride = is_draft ? a.drf_stride : a.tgt_stride;
  const int64_t row = is_draft ? drf_row(a, b, i) : tgt_row(a, b, i);
  const int lo = c * a.L.chunk1;
  const int hi = min(a.V, lo + a.L.chunk1);
  constexpr int W = BF16 ? 8 : 4;
  const bool vec_ok = (stride % W == 0) &&
                      ((reinterpret_cast<uintptr_t>(base) & (BF16 ? 15u : 15u)) == 0);
  float vals[kMaxPerThread];
  load_chunk<BF16>(base, row, stride, lo, hi, vec_ok, vals);

  Partial1 part;
  if (a.greedy) {
    float v = -INFINITY;
    int idx = 0x7fffffff;
#pragma unroll
    for (int it = 0; it < kMaxPerThread / W; ++it) {
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const int j = lo + (it * kThreads + static_cast<int>(threadIdx.x)) * W + e;
        if (j < hi) amax_merge(v, idx, vals[it * W + e], j);
      }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const float ov = __shfl_xor(v, m, 64);
      const int oi = __shfl_xor(idx, m, 64);
      amax_merge(v, idx, ov, oi);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
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
    m = block_max(m, shf);
    double s = 0.0;
    if (m > -INFINITY) {
#pragma unroll
      for (int e = 0; e < kMaxPerThread; ++e) s += static_cast<double>(expf(vals[e] - m));
    }
    s = block_sum(s, shd);
    part.m = m;
    part.idx = -1;
    part.s = s;
  }

  const int slots = 2 * a.gmax + 1;
  if (threadIdx.x == 0) {
    a.ws.part1[(static_cast<int64_t>(b) * slots + slot) * a.L.nch1 + c] = part;
    const int nrows = (g + 1) + ((a.greedy || a.draft_probs) ? 0 : g);
    const unsigned expected = static_cast<unsigned>(nrows * a.L.nch1);
    __threadfence();
    const unsigned prev = atomic_add_acq_rel(&a.ws.cnt1[b], 1u);
    last = (prev == expected - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  finalize_sequence<BF16>(a, b);
  if (threadIdx.x == 0) atomic_store_relaxed(&a.ws.cnt1[b], 0u);
}

// Resampling weight of element j (bit-identical wherever it is evaluated).
template <bool BF16>
__device__ __forceinline__ void weight_at(const Args& a, int64_t trow, int64_t drow, int j,
                                          const RowStat& rt, const RowStat& rq, int mode,
                                          float& w, float& p) {
  const float xt = ld<BF16>(a.tgt, trow, a.tgt_stride, j) * a.inv_t;
  p = static_cast<float>(static_cast<double>(expf(xt - rt.m)) / rt.s);
  if (mode == kModeBonus) {
    w = p;
    return;
  }
  float q;
  if (a.draft_probs) {
    q = static_cast<const float*>(a.drf)[drow * a.drf_stride + j];
  } else {
    const float xq = ld<BF16>(a.drf, drow, a.drf_stride, j) * a.inv_t;
    q = static_cast<float>(static_cast<double>(expf(xq - rq.m)) / rq.s);
  }
  w = fmaxf(p - q, 0.0f);
}

// Inclusive block scan of one fp64 value per thread (4 waves).
__device__ __forceinline__ double block_inclusive_scan(double v, double* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const double o = __shfl_up(v, m, 64);
    if (lane >= m) v += o;
  }
  if (lane == 63) sh[w] = v;
  __syncthreads();
  double off = 0.0;
  for (int q = 0; q < w; ++q) off += sh[q];
  __syncthreads();
  return off + v;
}

template <bool BF16>
__global__ __launch_bounds__(kThreads) void resample_kernel(Args a) {
  __shared__ double shd[4];
  __shared__ double shd2[4];
  __shared__ int last;
  __shared__ int sh_chunk;
  __shared__ double sh_acc, sh_tau, sh_total;
  __shared__ int sh_use_p;
  __shared__ int sh_tok_min;
  __shared__ float sh_margin;
  const int c = blockIdx.x, b = blockIdx.y;
  const int slots = 2 * a.gmax + 1;
  const Decision dec = a.ws.dec[b];
  const int k = dec.k;
  const int mode = dec.mode;
  const RowStat rt = a.ws.rows[static_cast<int64_t>(b) * slots + k];
  RowStat rq = rt;
  if (mode == kModeResidual && !a.draft_probs) rq = a.ws.rows[static_cast<int64_t>(b) * slots + a.gmax + 1 + k];
  const int64_t trow = tgt_row(a, b, k);
  const int64_t drow = mode == kModeResidual ? drf_row(a, b, k) : 0;

  const int lo = c * a.L.chunk2;
  const int hi = min(a.V, lo + a.L.chunk2);
  double sw = 0.0, sp = 0.0;
  for (int j = lo + threadIdx.x; j < hi; j += kThreads) {
    float w, p;
    weight_at<BF16>(a, trow, drow, j, rt, rq, mode, w, p);
    sw += static_cast<double>(w);
    sp += static_cast<double>(p);
  }
  sw = block_sum(sw, shd);
  sp = block_sum(sp, shd2);
  if (threadIdx.x == 0) {
    Partial2 pp;
    pp.w = sw;
    pp.p = sp;
    a.ws.part2[static_cast<int64_t>(b) * a.L.nch2 + c] = pp;
    __threadfence();
    const unsigned prev = atomic_add_acq_rel(&a.ws.cnt2[b], 1u);
    last = (prev == static_cast<unsigned>(a.L.nch2) - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();

  // ---- last block of sequence b: locate the chunk, then the element ----
  if (threadIdx.x == 0) {
    const Partial2* P = a.ws.part2 + static_cast<int64_t>(b) * a.L.nch2;
    double total = 0.0;
    for (int q = 0; q < a.L.nch2; ++q) total += load_agent(&P[q].w);
    int use_p = 0;
    if (mode == kModeResidual && !(total > 0.0)) {
      use_p = 1;  // residual sums to zero: fall back to p_k (engine/spec_decode.py:48)
      total = 0.0;
      for (int q = 0; q < a.L.nch2; ++q) total += load_agent(&P[q].p);
    }
    const double tau = static_cast<double>(a.u_res[b]) * total;
    double acc = 0.0;
    int chunk = -1, last_nonzero = 0;
    for (int q = 0; q < a.L.nch2; ++q) {
      const double sq = use_p ? load_agent(&P[q].p) : load_agent(&P[q].w);
      if (sq > 0.0) last_nonzero = q;
      if (acc + sq > tau) {
        chunk = q;
        break;
      }
      acc += sq;
    }
    if (chunk < 0) {  // tau within rounding of the total: take the last chunk with mass
      chunk = last_nonzero;
      acc = 0.0;
      for (int q = 0; q < chunk; ++q) acc += use_p ? load_agent(&P[q].p) : load_agent(&P[q].w);
    }
    sh_chunk = chunk;
    sh_acc = acc;
    sh_tau = tau;
    sh_total = total;
    sh_use_p = use_p;
    sh_tok_min = 0x7fffffff;
    sh_margin = 0.0f;
  }
  __syncthreads();
  const int chunk = sh_chunk;
  const double acc = sh_acc, tau = sh_tau, total = sh_total;
  const int use_p = sh_use_p;
  const int clo = chunk * a.L.chunk2;
  const int chi = min(a.V, clo + a.L.chunk2);
  const int per = (a.L.chunk2 + kThreads - 1) / kThreads;
  const int tlo = min(chi, clo + static_cast<int>(threadIdx.x) * per);
  const int thi = min(chi, tlo + per);
  double local = 0.0;
  for (int j = tlo; j < thi; ++j) {
    float w, p;
    weight_at<BF16>(a, trow, drow, j, rt, rq, mode, w, p);
    local += static_cast<double>(use_p ? p : w);
  }
  const double incl = block_inclusive_scan(local, shd);
  // Thread t owns [acc + incl_{t-1}, acc + incl_t); incl_{t-1} is read from the neighbour so
  // that exactly one thread claims tau.
  const double prev_incl = __shfl_up(incl, 1, 64);
  __shared__ double wave_last[4];
  if ((threadIdx.x & 63) == 63) wave_last[threadIdx.x >> 6] = incl;
  __syncthreads();
  double start;
  if (threadIdx.x == 0) {
    start = 0.0;
  } else if ((threadIdx.x & 63) == 0) {
    start = wave_last[(threadIdx.x >> 6) - 1];
  } else {
    start = prev_incl;
  }
  const bool claim = (acc + start <= tau) && (tau < acc + incl) && (thi > tlo);
  int tok = -1;
  float mg = 0.0f;
  if (claim) {
    double run = acc + start;
    int last_pos = -1;
    double lo_edge = run, hi_edge = run;
    for (int j = tlo; j < thi; ++j) {
      float w, p;
      weight_at<BF16>(a, trow, drow, j, rt, rq, mode, w, p);
      const double wj = static_cast<double>(use_p ? p : w);
      if (wj > 0.0) last_pos = j;
      const double nxt = run + wj;
      if (nxt > tau && wj > 0.0) {
        tok = j;
        lo_edge = run;
        hi_edge = nxt;
        break;
      }
      run = nxt;
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
  if (threadIdx.x == 0) {
    int pick = sh_tok_min == 0x7fffffff ? -1 : sh_tok_min;
    float pick_margin = sh_margin;
    if (pick < 0) {  // no thread claimed (rounding at the chunk end): last element with mass
      for (int j = chi - 1; j >= clo; --j) {
        float w, p;
        weight_at<BF16>(a, trow, drow, j, rt, rq, mode, w, p);
        if ((use_p ? p : w) > 0.0f) {
          pick = j;
          break;
        }
      }
      if (pick < 0) pick = clo;
      pick_margin = 0.0f;
    }
    a.out_tok[static_cast<int64_t>(b) * (a.gmax + 1) + k] = pick;
    if (a.margin) a.margin[b] = fminf(dec.margin, pick_margin);
    atomic_store_relaxed(&a.ws.cnt2[b], 0u);
  }
}

// softmax(x * inv_t) per row, written as fp32 probabilities: one block per row, three passes.
template <bool BF16>
__global__ __launch_bounds__(kThreads) void softmax_kernel(const void* x, int64_t in_stride, int V,
                                                           float inv_t, float* out,
                                                           int64_t out_stride) {
  __shared__ float shf[4];
  __shared__ double shd[4];
  const int64_t r = blockIdx.x;
  float m = -INFINITY;
  for (int j = threadIdx.x; j < V; j += kThreads) m = fmaxf(m, ld<BF16>(x, r, in_stride, j) * inv_t);
  m = block_max(m, shf);
  double s = 0.0;
  for (int j = threadIdx.x; j < V; j += kThreads)
    s += static_cast<double>(expf(ld<BF16>(x, r, in_stride, j) * inv_t - m));
  s = block_sum(s, shd);
  for (int j = threadIdx.x; j < V; j += kThreads) {
    const float xs = ld<BF16>(x, r, in_stride, j) * inv_t;
    out[r * out_stride + j] = static_cast<float>(static_cast<double>(expf(xs - m)) / s);
  }
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
  COOPT_REQUIRE(B <= kMaxCounters / 2, "B must be <= 65536");
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
  a.greedy = greedy ? 1 : 0;
  a.draft_probs = (draft_kind == 1) ? 1 : 0;
  a.B = B;
  a.gmax = gamma_max;
  a.V = V;
  a.L = make_layout(B, gamma_max, V);
  carve(&a.ws, reinterpret_cast<uintptr_t>(workspace), B, gamma_max, a.L);
  auto s = static_cast<hipStream_t>(stream);
  const bool bf16 = logits_dtype == COOPT_DT_BF16;
  const dim3 g1(a.L.nch1, 2 * gamma_max + 1, B);
  if (bf16)
    hipLaunchKernelGGL(row_stats_kernel<true>, g1, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(row_stats_kernel<false>, g1, dim3(kThreads), 0, s, a);
  int rc = coopt::check_launch("coopt_accept_sample/row_stats");
  if (rc != COOPT_OK || greedy) return rc;
  const dim3 g2(a.L.nch2, B);
  if (bf16)
    hipLaunchKernelGGL(resample_kernel<true>, g2, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(resample_kernel<false>, g2, dim3(kThreads), 0, s, a);
  return coopt::check_launch("coopt_accept_sample/resample");
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
  if (logits_dtype == COOPT_DT_BF16)
    hipLaunchKernelGGL(softmax_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                       logits, in_stride, V, inv_t, probs, out_stride);
  else
    hipLaunchKernelGGL(softmax_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                       logits, in_stride, V, inv_t, probs, out_stride);
  return coopt::check_launch("coopt_softmax");
}
