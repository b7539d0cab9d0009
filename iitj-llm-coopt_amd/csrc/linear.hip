// Weight-streaming linear layer for decode / verify row counts: Y[M, N] = X[M, K] W[N, K]^T
// in bf16 with fp32 accumulation, for M <= 256 (the 32-160 rows of a speculative step).
// Replaces torch.nn.functional.linear at the reference's projections (engine/model.py:238,
// 248, 250, 253: qkv, o, gate_up, down) and the logits projection.
//
// At these row counts the layer is a stream over W (2 bytes per weight, read once) with
// intensity M flop per weight byte (2M per weight), under the bf16 MFMA ridge (~310 flop/byte)
// for every M <= 256; the library GEMMs pick square macro tiles and leave most CUs idle on
// N = 4096 outputs.
//
// Decomposition.  A workgroup of WAVES waves owns WAVES * NW 16-column tiles of the output
// and a K range of `kt` elements; gridDim.y workgroups split K, and when it exceeds one they
// write fp32 partials that reduce_kernel sums in a fixed order (deterministic, no atomics).
//   * W streams from HBM straight into MFMA B operands: per 128-wide K step a lane reads 64
//     contiguous bytes of its output row as 4 x 16 B (MFMA j covers k0 + 32j + [8g, 8g+8),
//     g = lane / 16), PF steps ahead of the MFMAs.
//   * X is shared: each K step's [M, 128] slice is staged once per workgroup in LDS (double
//     buffered, rows padded to 272 bytes) and read by all waves as MFMA A operands.
//   * v_mfma_f32_16x16x32_bf16 with A = X rows, B = W rows: lane l holds
//     C[4(l/16) + i][l % 16] of each 16x16 tile.
//
// Tile-packed weights (coopt_linear_pack_weight).  W may instead be stored as [N/16][K/128]
// tiles of 16 rows x 128 K, each the 4 x 64 16-byte chunks in the order the lanes load them:
// chunk (j, l) = W[16 t + l % 16][128 u + 32 j + 8 (l / 16), +8).  A wave then reads each
// K step as 4 KB of consecutive bytes (1 KB per load instruction) instead of 16 rows x 256 B.
// The MFMA operands are the same as with row-major W, so the results are bit-identical;
// the packed stream measured 3-18 % faster on the verify and draft projections.
#include "common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kKB = 128;                  // K elements per step
constexpr int kPitch = kKB * 2 + 16;      // LDS bytes per staged X row

struct LinArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;
  int64_t ldw;
  int M, N, K;
  int kt;            // K elements per workgroup (multiple of kKB)
  uint16_t* y;
  int64_t ldy;
  float* part;       // [gridDim.y, 16 * MT, N] fp32 when gridDim.y > 1 or force_part
  int force_part;    // write fp32 partials even for a single K slice
};

// linear_kernel's scalar arguments, in order, from a LinArgs
#define LIN_ARGS(a) (a).x, (a).ldx, (a).w, (a).ldw, (a).M, (a).N, (a).K, (a).kt, (a).y, (a).ldy, \
                    (a).part, (a).force_part

__device__ __forceinline__ f32x4_t mfma_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4_t ldg16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// MT: 16-row tiles of M; NW: 16-column tiles per wave; WAVES: waves per workgroup;
// PF: K steps of W in flight per wave (even); PK: W is tile-packed; SILU: W is a gate_up
// weight packed with gate and up tiles interleaved (coopt_linear_pack_gate_up), K is not
// split, and the output is silu(gate) * up (F = N / 2 columns) instead of the projection.
// The arguments are scalars, not a LinArgs by value: the first sixteen kernel-argument dwords
// (x through ldy) are then preloaded into SGPRs (the build's kernarg-preload option), so the
// first X / W loads do not wait for a kernel-argument load; part and force_part, needed only
// at the end, load from the segment.
template <int MT, int NW, int WAVES, int PF, bool PK, bool SILU = false>
__global__ __launch_bounds__(64 * WAVES) void linear_kernel(
    const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw, int M, int N, int K, int kt,
    uint16_t* y, int64_t ldy, float* part, int force_part) {
  const LinArgs a{x, ldx, w, ldw, M, N, K, kt, y, ldy, part, force_part};
  static_assert(!SILU || (PK && NW == 1 && WAVES % 2 == 0), "gate / up tile pairs per wave pair");
  static_assert(PF % 2 == 0, "the step loop is unrolled by PF and alternates X buffers");
  constexpr int kThreads = 64 * WAVES;
  constexpr int kRowsPerRound = kThreads / 16;                     // X rows staged per round
  constexpr int kRounds = (MT * 16 + kRowsPerRound - 1) / kRowsPerRound;
  __shared__ __attribute__((aligned(16))) unsigned char xs[2][MT * 16 * kPitch];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * WAVES + wave) * NW * 16;
  const int kbeg = blockIdx.y * a.kt;
  const int nsteps = (a.K - kbeg < a.kt ? a.K - kbeg : a.kt) / kKB;
  const int last = nsteps - 1;

  // W of this lane (clamped into [0, N): columns past N are computed and dropped).  Row-major:
  // the lane's row at K offset 8g, chunk j of a step 32j further.  Packed: the lane's chunk of
  // its 16-column tile at the slice's first K step, chunk j of a step 64 lanes further.
  constexpr int kWStep = PK ? 16 * kKB : kKB;  // elements from one K step to the next
  constexpr int kWChunk = PK ? 64 * 8 : 32;    // elements from chunk j to chunk j + 1
  const uint16_t* wrow[NW];
#pragma unroll
  for (int nt = 0; nt < NW; ++nt) {
    if constexpr (PK) {
      int ct = (n0 + nt * 16) / 16;
      ct = ct < a.N / 16 ? ct : a.N / 16 - 1;
      wrow[nt] = a.w + (static_cast<int64_t>(ct) * (a.K / kKB) + kbeg / kKB) * (16 * kKB) + lane * 8;
    } else {
      int n = n0 + nt * 16 + l16;
      n = n < a.N ? n : a.N - 1;
      wrow[nt] = a.w + static_cast<int64_t>(n) * a.ldw + kbeg + 8 * g;
    }
  }
  // X staging: in round r, thread t loads 16 B of row r * kRowsPerRound + t / 16 at byte
  // 16 (t % 16) of the step; rows >= 16 MT are not staged.  Rows in [M, 16 MT) repeat row
  // M - 1: their outputs are never stored, and an unconditional load keeps the compiler's
  // load counting exact (a load under a branch makes it wait for every load in flight).
  const int xr_row = threadIdx.x >> 4, xr_col = (threadIdx.x & 15) * 8;
  const uint16_t* xrow[kRounds];
  bool xin[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int m = r * kRowsPerRound + xr_row;
    xin[r] = m < MT * 16;
    xrow[r] = a.x + static_cast<int64_t>(m < a.M ? m : a.M - 1) * a.ldx + kbeg + xr_col;
  }

  auto load_x = [&](int s, u32x4_t (&xr)[kRounds]) {
#pragma unroll
    for (int r = 0; r < kRounds; ++r) xr[r] = ldg16(xrow[r] + s * kKB);
  };
  auto load_w = [&](int s, u32x4_t (&wr)[NW][4]) {
#pragma unroll
    for (int nt = 0; nt < NW; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) wr[nt][j] = ldg16(wrow[nt] + s * kWStep + kWChunk * j);
  };
  auto store_x = [&](int buf, const u32x4_t (&xr)[kRounds]) {
#pragma unroll
    for (int r = 0; r < kRounds; ++r)
      if (xin[r])
        *reinterpret_cast<u32x4_t*>(
            &xs[buf][(r * kRowsPerRound + xr_row) * kPitch + xr_col * 2]) = xr[r];
  };

  f32x4_t acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NW; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // A fragments of MFMA group j + 1 are read from LDS while group j's MFMAs run, so no MFMA
  // waits on the latency of the read that feeds it.
  auto read_frag = [&](int buf, int j, u32x4_t (&fa)[MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      fa[mt] = *reinterpret_cast<const u32x4_t*>(
          &xs[buf][(mt * 16 + l16) * kPitch + 64 * j + 16 * g]);
  };
  auto mfma_group = [&](int j, const u32x4_t (&fa)[MT], const u32x4_t (&wr)[NW][4]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NW; ++nt) acc[mt][nt] = mfma_bf16(fa[mt], wr[nt][j], acc[mt][nt]);
  };
  // (sched_barrier keeps the scheduler from sinking the reads back next to their MFMAs)
  auto compute = [&](int buf, const u32x4_t (&wr)[NW][4]) {
    u32x4_t f0[MT], f1[MT];
    read_frag(buf, 0, f0);
    read_frag(buf, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(0, f0, wr);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(buf, 2, f0);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(1, f1, wr);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(buf, 3, f1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(2, f0, wr);
    mfma_group(3, f1, wr);
  };

  // Pipeline.  W: a ring of PF register buffers, step s + PF loaded right after step s's
  // MFMAs.  X: two register buffers, step s + 2 loaded at the start of step s and stored to
  // LDS at the end of step s + 1, so the wait for it never covers the W loads issued after
  // it.  Step indices past the last are clamped: those reloads hit L2, not HBM, and keep
  // every load unconditional.
  u32x4_t xq[2][kRounds];
  u32x4_t wbuf[PF][NW][4];
  load_x(0, xq[0]);
  load_x(last < 1 ? last : 1, xq[1]);
#pragma unroll
  for (int p = 0; p < PF; ++p) load_w(p < last ? p : last, wbuf[p]);
  store_x(0, xq[0]);
  for (int s0 = 0; s0 < nsteps; s0 += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int s = s0 + u;
      if (s < nsteps) {
        load_x(s + 2 < last ? s + 2 : last, xq[u & 1]);
        __syncthreads();
        compute(u & 1, wbuf[u]);
        load_w(s + PF < last ? s + PF : last, wbuf[u]);
        store_x((u + 1) & 1, xq[(u + 1) & 1]);
      }
    }
  }

  // Epilogue: lane holds rows 16 mt + 4 g + i of column n0 + 16 nt + l16.
  if constexpr (SILU) {
    // Wave 2p holds gate tile t = blockIdx.x * WAVES / 2 + p and wave 2p + 1 the matching up
    // tile; the up wave hands its sums over through LDS (the X staging is dead by now).  Each
    // sum is rounded to bf16 first -- the projection's output -- then silu(gate) * up as
    // silu_mul_kernel computes it, rounded once more.
    __syncthreads();
    float* xch = reinterpret_cast<float*>(&xs[0][0]);
    const int pair = wave >> 1;
    if (wave & 1) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) xch[((pair * MT + mt) * 4 + i) * 64 + lane] = acc[mt][0][i];
    }
    __syncthreads();
    if (wave & 1) return;
    const int F = a.N / 2;
    const int j = (blockIdx.x * (WAVES / 2) + pair) * 16 + l16;
    if (j >= F) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mt * 16 + 4 * g + i;
        if (m >= a.M) continue;
        const float gv = bf16_to_f32(f32_to_bf16(acc[mt][0][i]));
        const float uv = bf16_to_f32(f32_to_bf16(xch[((pair * MT + mt) * 4 + i) * 64 + lane]));
        a.y[static_cast<int64_t>(m) * a.ldy + j] = f32_to_bf16(gv / (1.0f + __expf(-gv)) * uv);
      }
    return;
  }
  if (gridDim.y == 1 && !a.force_part) {
#pragma unroll
    for (int nt = 0; nt < NW; ++nt) {
      const int n = n0 + nt * 16 + l16;
      if (n >= a.N) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mt * 16 + 4 * g + i;
          if (m < a.M) a.y[static_cast<int64_t>(m) * a.ldy + n] = f32_to_bf16(acc[mt][nt][i]);
        }
    }
  } else {
    float* p = a.part + static_cast<int64_t>(blockIdx.y) * (MT * 16) * a.N;
#pragma unroll
    for (int nt = 0; nt < NW; ++nt) {
      const int n = n0 + nt * 16 + l16;
      if (n >= a.N) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p[static_cast<int64_t>(mt * 16 + 4 * g + i) * a.N + n] = acc[mt][nt][i];
    }
  }
}

// y[m, n] = bf16(sum over slices s = 0..ks-1, in order, of part[s, m, n]); 4 columns a thread.
// KS: compile-time bound on ks (all loads issued before the first add), 0 = runtime bound.
template <int KS>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ part, int ks,
                                                     int64_t slice, int M, int N,
                                                     uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int nq = N / 4;
  if (gid >= static_cast<int64_t>(M) * nq) return;
  const int m = static_cast<int>(gid / nq), n = static_cast<int>(gid % nq) * 4;
  const float* p = part + static_cast<int64_t>(m) * N + n;
  float4 s;
  if constexpr (KS > 0) {
    Partials4<KS> pl;
    pl.load(p, ks, slice);
    s = pl.sum(ks);
  } else {
    s = sum_partials4(p, ks, slice);
  }
  uint16_t* o = y + static_cast<int64_t>(m) * ldy + n;
  const uint32_t lo = f32_to_bf16(s.x) | (static_cast<uint32_t>(f32_to_bf16(s.y)) << 16);
  const uint32_t hi = f32_to_bf16(s.z) | (static_cast<uint32_t>(f32_to_bf16(s.w)) << 16);
  *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
}

struct Plan {
  int mt, nw, waves, ks, kt;
};

// 16-row tiles of M, rounded up to an instantiated count.
int m_tiles(int M) {
  const int t = (M + 15) / 16;
  static const int kTiles[] = {1, 2, 4, 6, 8, 10, 12, 16};
  for (int v : kTiles)
    if (t <= v) return v;
  return -1;
}

// Launch shape (measured on MI355X over the decode / verify projections of an 8B / 1B Llama
// pair, both weight layouts): 8 waves of one 16-column tile each, or 4 waves at M <= 64 below
// lm_head widths (the draft's 16384-wide gate_up: 15.0 us packed / 18.6 us row-major against
// 19.0 us with 8 waves and K split twice), or 4 column tiles per wave for very wide N
// (lm_head).  K is split in powers of two while the grid stays within 256 workgroups and each
// keeps at least 4 K steps; every split adds 4 * 16 * MT bytes of fp32 partials per column
// against 2 * kt bytes of weights.
Plan plan_for(int M, int N, int K) {
  Plan p{m_tiles(M), 1, 8, 1, K};
  if (p.mt <= 4 && N < 65536) p.waves = 4;
  if (p.mt <= 4 && N >= 65536) p.nw = 4;
  // 16 row tiles, or 4 row tiles with 4 column tiles per wave, exceed two waves' registers
  // per SIMD (they spilled to scratch): 4-wave blocks, one wave per SIMD, hold them.
  if (p.mt == 16 || (p.mt == 4 && p.nw == 4)) p.waves = 4;
  const int steps = K / kKB;
  auto split_for = [&](int waves) {  // K splits for `waves` waves of p.nw column tiles
    const int nb = (N + waves * p.nw * 16 - 1) / (waves * p.nw * 16);
    int k = 1;
    while (k < 16 && nb * k * 2 <= 256 && steps / (k * 2) >= 4) k *= 2;
    return k;
  };
  int ks = split_for(p.waves);
  // 160 rows: 7 waves (112 columns) where that fills more of the 256 CUs than 8 do -- the
  // target's qkv, N = 6144: 55 x 4 = 220 workgroups against 48 x 4 = 192, 22.2 -> 20.5 us
  if (p.mt == 10 && p.nw == 1 && p.waves == 8) {
    const int k7 = split_for(7);
    if (((N + 111) / 112) * k7 > ((N + 127) / 128) * ks && ((N + 111) / 112) * k7 <= 256) {
      p.waves = 7;
      ks = k7;
    }
  }
  p.kt = ((steps + ks - 1) / ks) * kKB;
  p.ks = (K + p.kt - 1) / p.kt;
  return p;
}

template <int MT, int NW, int WAVES, int PF>
void launch_cfg(const Plan& p, const LinArgs& a, bool packed, hipStream_t s) {
  const int cols = WAVES * NW * 16;
  const dim3 grid((a.N + cols - 1) / cols, p.ks);
  if (packed)
    hipLaunchKernelGGL((linear_kernel<MT, NW, WAVES, PF, true>), grid, dim3(64 * WAVES), 0, s, LIN_ARGS(a));
  else
    hipLaunchKernelGGL((linear_kernel<MT, NW, WAVES, PF, false>), grid, dim3(64 * WAVES), 0, s, LIN_ARGS(a));
}

template <int MT>
void launch_mt(const Plan& p, const LinArgs& a, bool packed, hipStream_t s) {
  if constexpr (MT == 16) {
    launch_cfg<MT, 1, 4, 2>(p, a, packed, s);
  } else {
    if constexpr (MT <= 4) {
      if (p.nw == 4) {
        if constexpr (MT == 4) {
          launch_cfg<MT, 4, 4, 2>(p, a, packed, s);
        } else {
          launch_cfg<MT, 4, 8, 2>(p, a, packed, s);
        }
        return;
      }
      if (p.waves == 4) return launch_cfg<MT, 1, 4, 2>(p, a, packed, s);
    }
    if constexpr (MT == 10) {
      if (p.waves == 7) return launch_cfg<MT, 1, 7, 2>(p, a, packed, s);
    }
    launch_cfg<MT, 1, 8, 2>(p, a, packed, s);
  }
}

// Tile packing: thread o writes 16-byte chunk o of the packed layout, reading it from the
// row-major weight.  Chunk o = ((t * (K/128) + u) * 4 + j) * 64 + l.
// With gu_half = F (a gate_up weight of 2F rows), packed tile 2s holds gate rows
// [16 s, 16 s + 16) and tile 2s + 1 up rows [F + 16 s, F + 16 s + 16).
__global__ __launch_bounds__(256) void pack_kernel(const uint16_t* __restrict__ w, int64_t ldw,
                                                  int kt, int64_t chunks, int gu_half,
                                                  uint16_t* __restrict__ out) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= chunks) return;
  const int l = static_cast<int>(o & 63), j = static_cast<int>((o >> 6) & 3);
  const int64_t tu = o >> 8;
  const int64_t t = tu / kt;
  const int u = static_cast<int>(tu - t * kt);
  const int64_t src_t = gu_half ? ((t & 1) ? gu_half / 16 + (t >> 1) : (t >> 1)) : t;
  const int64_t row = 16 * src_t + (l & 15);
  const int64_t col = static_cast<int64_t>(kKB) * u + 32 * j + 8 * (l >> 4);
  *reinterpret_cast<u32x4_t*>(out + o * 8) = ldg16(w + row * ldw + col);
}

}  // namespace

extern "C" size_t coopt_linear_workspace(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % kKB != 0 || m_tiles(M) < 0) return 0;
  const Plan p = plan_for(M, N, K);
  return p.ks > 1 ? static_cast<size_t>(p.ks) * p.mt * 16 * N * sizeof(float) : 0;
}

namespace {

// Shared by coopt_linear and coopt_linear_partials: checks, then the split-K launch.  With
// `partials` every slice (also a single one) goes to the workspace as fp32.
int run_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K,
               void* y, int64_t ldy, void* workspace, size_t workspace_bytes, bool partials,
               bool packed, hipStream_t s, Plan& p);

// The fixed-order reduction of coopt_linear's ks > 1 slices into y.
int reduce_into(const Plan& p, int M, int N, const void* workspace, void* y, int64_t ldy,
                hipStream_t s, const char* who);

}  // namespace

extern "C" int coopt_linear_split(int M, int N, int K, int* ks, int* rows_padded) {
  coopt::clear_error();
  COOPT_REQUIRE(ks && rows_padded, "null output pointer");
  COOPT_REQUIRE(M > 0 && M <= 256 && N > 0 && K > 0 && K % kKB == 0, "unsupported shape");
  const Plan p = plan_for(M, N, K);
  *ks = p.ks;
  *rows_padded = p.mt * 16;
  return COOPT_OK;
}

extern "C" int coopt_linear_partials(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     int M, int N, int K, void* workspace,
                                     size_t workspace_bytes, coopt_stream_t stream) {
  coopt::clear_error();
  Plan p{};
  return run_linear(x, ldx, w, ldw, M, N, K, nullptr, 0, workspace, workspace_bytes, true,
                    false, reinterpret_cast<hipStream_t>(stream), p);
}

extern "C" int coopt_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N,
                            int K, void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                            coopt_stream_t stream) {
  coopt::clear_error();
  Plan p{};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc = run_linear(x, ldx, w, ldw, M, N, K, y, ldy, workspace, workspace_bytes, false, false,
                      s, p);
  if (rc != COOPT_OK || M == 0 || N == 0 || p.ks == 1) return rc;
  return reduce_into(p, M, N, workspace, y, ldy, s, "coopt_linear");
}

namespace {

int pack_weight(const void* w, int64_t ldw, int N, int K, int gu_half, void* out,
                coopt_stream_t stream, const char* who) {
  COOPT_REQUIRE(N >= 0 && K >= 0, "negative size");
  if (N == 0 || K == 0) return COOPT_OK;
  COOPT_REQUIRE(N % 16 == 0 && K % kKB == 0, "N must be a multiple of 16 and K of 128");
  COOPT_REQUIRE(gu_half == 0 || (N == 2 * gu_half && gu_half % 16 == 0),
                "a gate_up weight has 2F rows with F a multiple of 16");
  COOPT_REQUIRE(w && out, "null pointer");
  COOPT_REQUIRE(coopt::aligned16(w) && coopt::aligned16(out), "w and out must be 16-byte aligned");
  COOPT_REQUIRE(ldw >= K && ldw % 8 == 0, "row stride of w must be >= K and a multiple of 8");
  COOPT_REQUIRE(static_cast<int64_t>(N) * ldw < (int64_t(1) << 62), "w too large");
  const int64_t chunks = static_cast<int64_t>(N) * (K / 8);
  COOPT_REQUIRE((chunks + 255) / 256 <= 0x7fffffff, "w too large");
  hipLaunchKernelGGL(pack_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), ldw,
                     K / kKB, chunks, gu_half, static_cast<uint16_t*>(out));
  return coopt::check_launch(who);
}

template <int MT, int WAVES>
void launch_silu(int F, const LinArgs& a, hipStream_t s) {
  // WAVES / 2 (gate, up) tile pairs per workgroup; pairs of a trailing partial workgroup past
  // the weight read clamped tiles and write nothing (their columns are >= F)
  const int rows = 16 * WAVES;
  hipLaunchKernelGGL((linear_kernel<MT, 1, WAVES, 2, true, true>), dim3((2 * F + rows - 1) / rows, 1),
                     dim3(64 * WAVES), 0, s, LIN_ARGS(a));
}

}  // namespace

extern "C" int coopt_linear_pack_weight(const void* w, int64_t ldw, int N, int K, void* out,
                                        coopt_stream_t stream) {
  coopt::clear_error();
  return pack_weight(w, ldw, N, K, 0, out, stream, "coopt_linear_pack_weight");
}

extern "C" int coopt_linear_pack_gate_up(const void* w, int64_t ldw, int F, int K, void* out,
                                         coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(F >= 0, "negative size");
  return pack_weight(w, ldw, 2 * F, K, F, out, stream, "coopt_linear_pack_gate_up");
}

extern "C" int coopt_linear_silu_supported(int M, int F, int K) {
  if (M <= 0 || F <= 0 || K <= 0 || F % 16 || K % kKB || M > 256 || m_tiles(M) < 0 ||
      2LL * F >= 65536)
    return 0;
  const Plan p = plan_for(M, 2 * F, K);
  return p.ks == 1 && p.nw == 1 && (p.waves == 4 ? p.mt <= 4 : p.mt == 10) ? 1 : 0;
}

extern "C" int coopt_linear_silu_packed(const void* x, int64_t ldx, const void* w_gu_packed,
                                        int M, int F, int K, void* y, int64_t ldy,
                                        coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(M >= 0 && F >= 0 && K >= 0, "negative size");
  if (M == 0 || F == 0) return COOPT_OK;
  COOPT_REQUIRE(coopt_linear_silu_supported(M, F, K),
                "shape outside the fused gate_up + SiLU path (M <= 64 or 129-160, F a multiple "
                "of 16, 2F < 65536, K a multiple of 128 without a K split)");
  COOPT_REQUIRE(x && w_gu_packed && y, "null pointer");
  COOPT_REQUIRE(coopt::aligned16(x) && coopt::aligned16(w_gu_packed), "x and w must be 16-byte aligned");
  COOPT_REQUIRE(ldx >= K && ldx % 8 == 0, "row stride of x must be >= K and a multiple of 8");
  COOPT_REQUIRE(ldy >= F, "row stride of y must be >= F");
  const Plan p = plan_for(M, 2 * F, K);
  LinArgs a{static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(w_gu_packed), K, M,
            2 * F, K, p.kt, static_cast<uint16_t*>(y), ldy, nullptr, 0};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (p.mt) {
    case 1: launch_silu<1, 4>(F, a, s); break;
    case 2: launch_silu<2, 4>(F, a, s); break;
    case 4: launch_silu<4, 4>(F, a, s); break;
    default: launch_silu<10, 8>(F, a, s); break;   // the verify rows (129-160), 8 waves
  }
  return coopt::check_launch("coopt_linear_silu_packed");
}

extern "C" int coopt_linear_packed(const void* x, int64_t ldx, const void* w_packed, int M, int N,
                                   int K, void* y, int64_t ldy, void* workspace,
                                   size_t workspace_bytes, coopt_stream_t stream) {
  coopt::clear_error();
  Plan p{};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc = run_linear(x, ldx, w_packed, K, M, N, K, y, ldy, workspace, workspace_bytes, false,
                      true, s, p);
  if (rc != COOPT_OK || M == 0 || N == 0 || p.ks == 1) return rc;
  return reduce_into(p, M, N, workspace, y, ldy, s, "coopt_linear_packed");
}

extern "C" int coopt_linear_partials_packed(const void* x, int64_t ldx, const void* w_packed,
                                            int M, int N, int K, void* workspace,
                                            size_t workspace_bytes, coopt_stream_t stream) {
  coopt::clear_error();
  Plan p{};
  return run_linear(x, ldx, w_packed, K, M, N, K, nullptr, 0, workspace, workspace_bytes, true,
                    true, reinterpret_cast<hipStream_t>(stream), p);
}

namespace {

int reduce_into(const Plan& p, int M, int N, const void* workspace, void* y, int64_t ldy,
                hipStream_t s, const char* who) {
  const int64_t n4 = static_cast<int64_t>(M) * (N / 4);
  const dim3 grid(static_cast<unsigned>((n4 + 255) / 256));
  const float* part = static_cast<const float*>(workspace);
  const int64_t slice = static_cast<int64_t>(p.mt) * 16 * N;
  uint16_t* yp = static_cast<uint16_t*>(y);
  switch (partials_bound(p.ks)) {
    case 2: hipLaunchKernelGGL(reduce_kernel<2>, grid, dim3(256), 0, s, part, p.ks, slice, M, N, yp, ldy); break;
    case 4: hipLaunchKernelGGL(reduce_kernel<4>, grid, dim3(256), 0, s, part, p.ks, slice, M, N, yp, ldy); break;
    case 8: hipLaunchKernelGGL(reduce_kernel<8>, grid, dim3(256), 0, s, part, p.ks, slice, M, N, yp, ldy); break;
    case 16: hipLaunchKernelGGL(reduce_kernel<16>, grid, dim3(256), 0, s, part, p.ks, slice, M, N, yp, ldy); break;
    default: hipLaunchKernelGGL(reduce_kernel<0>, grid, dim3(256), 0, s, part, p.ks, slice, M, N, yp, ldy); break;
  }
  return coopt::check_launch(who);
}

int run_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K,
               void* y, int64_t ldy, void* workspace, size_t workspace_bytes, bool partials,
               bool packed, hipStream_t s, Plan& p) {
  COOPT_REQUIRE(M >= 0 && N >= 0 && K >= 0, "negative size");
  if (M == 0 || N == 0) return COOPT_OK;
  COOPT_REQUIRE(M <= 256, "M must be <= 256 (decode / verify row counts)");
  COOPT_REQUIRE(K > 0 && K % kKB == 0, "K must be a positive multiple of 128");
  COOPT_REQUIRE(N % 4 == 0, "N must be a multiple of 4");
  COOPT_REQUIRE(!packed || N % 16 == 0, "packed weights need N a multiple of 16");
  COOPT_REQUIRE(x && w && (y || partials), "null pointer");
  COOPT_REQUIRE(coopt::aligned16(x) && coopt::aligned16(w), "x and w must be 16-byte aligned");
  COOPT_REQUIRE(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0,
                "row strides of x and w must be >= K and multiples of 8");
  COOPT_REQUIRE(partials || (ldy >= N && ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0),
                "y rows must be 8-byte aligned with stride >= N, a multiple of 4");
  COOPT_REQUIRE(static_cast<int64_t>(N) * ldw < (int64_t(1) << 62), "w too large");
  p = plan_for(M, N, K);
  if (packed && N >= 65536 && p.mt <= 4 && p.ks == 1) {
    // lm_head widths from packed weights stream best with one column tile per wave (32 rows:
    // 98.8 us, 4 waves; 64 rows: 107.1 us, 8 waves; against 107.1 / 119+ us with 4 tiles per
    // wave).  The split (ks = 1) and so the workspace and partial layout are unchanged.
    p.nw = 1;
    p.waves = p.mt <= 2 ? 4 : 8;
  }
  const size_t need = partials ? static_cast<size_t>(p.ks) * p.mt * 16 * N * sizeof(float)
                               : coopt_linear_workspace(M, N, K);
  COOPT_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr) &&
                    (need == 0 || coopt::aligned16(workspace)),
                "workspace smaller than required (or misaligned)");
  LinArgs a{static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(w), ldw, M, N, K,
            p.kt, static_cast<uint16_t*>(y), ldy, static_cast<float*>(workspace)};
  a.force_part = partials ? 1 : 0;  // fp32 slices even when K is not split
  switch (p.mt) {
    case 1: launch_mt<1>(p, a, packed, s); break;
    case 2: launch_mt<2>(p, a, packed, s); break;
    case 4: launch_mt<4>(p, a, packed, s); break;
    case 6: launch_mt<6>(p, a, packed, s); break;
    case 8: launch_mt<8>(p, a, packed, s); break;
    case 10: launch_mt<10>(p, a, packed, s); break;
    case 12: launch_mt<12>(p, a, packed, s); break;
    default: launch_mt<16>(p, a, packed, s); break;
  }
  return coopt::check_launch(partials ? (packed ? "coopt_linear_partials_packed" : "coopt_linear_partials")
                                      : (packed ? "coopt_linear_packed" : "coopt_linear"));
}

}  // namespace
