// Elementwise stages of the Llama forward around the verify path, fused the way the
// reference's forward fuses them (engine/model.py:234-254, vLLM's rms_norm /
// fused_add_rms_norm / rotary_embedding / silu_and_mul): one launch per stage instead of the
// chain of small elementwise kernels plain torch issues.
#include "common.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum_f32(float v, float* sh) {
  v = wave_sum_f32(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint16_t round_bf16(float f) { return f32_to_bf16(f); }

// One block per row.  With a residual: r = bf16(x + residual), residual := r.  Then
// out = bf16(w * bf16(r * rsqrt(mean(r^2) + eps))) -- the rounding points of
// `w * (x.float() * rsqrt(...)).to(bf16)` (engine/model.py:85-89).
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                            uint16_t* __restrict__ residual,
                                                            const uint16_t* __restrict__ w,
                                                            uint16_t* __restrict__ out, int H,
                                                            float eps) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * H;
  uint16_t* rr = residual ? residual + row * H : nullptr;
  float ss = 0.0f;
  for (int i = threadIdx.x * 8; i < H; i += kThreads * 8) {
    const uint4 xv = *reinterpret_cast<const uint4*>(xr + i);
    uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    if (rr) {
      const uint4 rv = *reinterpret_cast<const uint4*>(rr + i);
      const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = bf16_to_f32(static_cast<uint16_t>(xw[e])) + bf16_to_f32(static_cast<uint16_t>(rw[e]));
        const float a1 = bf16_to_f32(static_cast<uint16_t>(xw[e] >> 16)) + bf16_to_f32(static_cast<uint16_t>(rw[e] >> 16));
        xw[e] = round_bf16(a0) | (static_cast<uint32_t>(round_bf16(a1)) << 16);
      }
      *reinterpret_cast<uint4*>(rr + i) = make_uint4(xw[0], xw[1], xw[2], xw[3]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = bf16_to_f32(static_cast<uint16_t>(xw[e]));
      const float a1 = bf16_to_f32(static_cast<uint16_t>(xw[e] >> 16));
      ss += a0 * a0 + a1 * a1;
    }
  }
  const float rs = rsqrtf(block_sum_f32(ss, sh) / static_cast<float>(H) + eps);
  const uint16_t* src = rr ? rr : xr;
  for (int i = threadIdx.x * 8; i < H; i += kThreads * 8) {
    const uint4 xv = *reinterpret_cast<const uint4*>(src + i);
    const uint4 wv = *reinterpret_cast<const uint4*>(w + i);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float n0 = bf16_to_f32(round_bf16(bf16_to_f32(static_cast<uint16_t>(xw[e])) * rs));
      const float n1 = bf16_to_f32(round_bf16(bf16_to_f32(static_cast<uint16_t>(xw[e] >> 16)) * rs));
      const float y0 = bf16_to_f32(static_cast<uint16_t>(ww[e])) * n0;
      const float y1 = bf16_to_f32(static_cast<uint16_t>(ww[e] >> 16)) * n1;
      ow[e] = round_bf16(y0) | (static_cast<uint32_t>(round_bf16(y1)) << 16);
    }
    *reinterpret_cast<uint4*>(out + row * H + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

// The same stage with the row held in registers: one read of x (and the residual) and of w,
// issued together, one block reduction, then the normalisation from registers -- a single
// global round trip for the short rows of decode and verify steps.  CPT 8-element chunks per
// thread cover H <= CPT * 8 * kThreads.
// With `part` set, x is not read: x[row] = bf16(sum of the ks fp32 slices part[k * slice +
// row * H]) -- the split-K partials of the producing linear layer, reduced here in the order
// its own reduction uses, so the result is the same as reducing first.
template <int CPT>
__global__ __launch_bounds__(kThreads) void rms_norm_reg_kernel(const uint16_t* __restrict__ x,
                                                                uint16_t* __restrict__ residual,
                                                                const uint16_t* __restrict__ w,
                                                                uint16_t* __restrict__ out,
                                                                int H, float eps,
                                                                const float* __restrict__ part,
                                                                int ks, int64_t slice) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * H;
  uint16_t* rr = residual ? residual + row * H : nullptr;
  uint32_t xw[CPT][4], ww[CPT][4];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int i = (c * kThreads + threadIdx.x) * 8;
    if (i >= H) continue;
    const uint4 wv = *reinterpret_cast<const uint4*>(w + i);
    if (part) {
      const float* pr = part + row * H + i;
      const float4 lo = sum_partials4(pr, ks, slice), hi = sum_partials4(pr + 4, ks, slice);
      xw[c][0] = round_bf16(lo.x) | (static_cast<uint32_t>(round_bf16(lo.y)) << 16);
      xw[c][1] = round_bf16(lo.z) | (static_cast<uint32_t>(round_bf16(lo.w)) << 16);
      xw[c][2] = round_bf16(hi.x) | (static_cast<uint32_t>(round_bf16(hi.y)) << 16);
      xw[c][3] = round_bf16(hi.z) | (static_cast<uint32_t>(round_bf16(hi.w)) << 16);
    } else {
      const uint4 xv = *reinterpret_cast<const uint4*>(xr + i);
      xw[c][0] = xv.x; xw[c][1] = xv.y; xw[c][2] = xv.z; xw[c][3] = xv.w;
    }
    ww[c][0] = wv.x; ww[c][1] = wv.y; ww[c][2] = wv.z; ww[c][3] = wv.w;
    if (rr) {
      const uint4 rv = *reinterpret_cast<const uint4*>(rr + i);
      const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = bf16_to_f32(static_cast<uint16_t>(xw[c][e])) + bf16_to_f32(static_cast<uint16_t>(rw[e]));
        const float a1 = bf16_to_f32(static_cast<uint16_t>(xw[c][e] >> 16)) + bf16_to_f32(static_cast<uint16_t>(rw[e] >> 16));
        xw[c][e] = round_bf16(a0) | (static_cast<uint32_t>(round_bf16(a1)) << 16);
      }
      *reinterpret_cast<uint4*>(rr + i) = make_uint4(xw[c][0], xw[c][1], xw[c][2], xw[c][3]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = bf16_to_f32(static_cast<uint16_t>(xw[c][e]));
      const float a1 = bf16_to_f32(static_cast<uint16_t>(xw[c][e] >> 16));
      ss += a0 * a0 + a1 * a1;
    }
  }
  const float rs = rsqrtf(block_sum_f32(ss, sh) / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int i = (c * kThreads + threadIdx.x) * 8;
    if (i >= H) continue;
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float n0 = bf16_to_f32(round_bf16(bf16_to_f32(static_cast<uint16_t>(xw[c][e])) * rs));
      const float n1 = bf16_to_f32(round_bf16(bf16_to_f32(static_cast<uint16_t>(xw[c][e] >> 16)) * rs));
      const float y0 = bf16_to_f32(static_cast<uint16_t>(ww[c][e])) * n0;
      const float y1 = bf16_to_f32(static_cast<uint16_t>(ww[c][e] >> 16)) * n1;
      ow[e] = round_bf16(y0) | (static_cast<uint32_t>(round_bf16(y1)) << 16);
    }
    *reinterpret_cast<uint4*>(out + row * H + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

// rms_norm_reg_kernel's partials path with the slice count bounded at compile time (KS):
// every load of the row -- w, the residual and the KS partial slices of each chunk -- is
// issued before the first add, so the row costs one global round trip.  Same arithmetic and
// order as rms_norm_reg_kernel, so the same result.  The residual is required (the fused
// add that follows every projection reduced this way).
template <int CPT, int KS>
__global__ __launch_bounds__(kThreads) void rms_norm_part_kernel(uint16_t* __restrict__ residual,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ out, int H,
                                                                 float eps,
                                                                 const float* __restrict__ part,
                                                                 int ks, int64_t slice) {
  __shared__ float sh[4];
  const int64_t row = blockIdx.x;
  uint16_t* rr = residual + row * H;
  Partials4<KS> plo[CPT], phi[CPT];
  uint4 wv[CPT], rv[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int i = (c * kThreads + threadIdx.x) * 8;
    const int il = i < H ? i : H - 8;  // past-the-row chunks load the last one, never stored
    wv[c] = *reinterpret_cast<const uint4*>(w + il);
    rv[c] = *reinterpret_cast<const uint4*>(rr + il);
    const float* pr = part + row * H + il;
    plo[c].load(pr, ks, slice);
    phi[c].load(pr + 4, ks, slice);
  }
  uint32_t xw[CPT][4];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int i = (c * kThreads + threadIdx.x) * 8;
    const float4 lo = plo[c].sum(ks), hi = phi[c].sum(ks);
    xw[c][0] = round_bf16(lo.x) | (static_cast<uint32_t>(round_bf16(lo.y)) << 16);
    xw[c][1] = round_bf16(lo.z) | (static_cast<uint32_t>(round_bf16(lo.w)) << 16);
    xw[c][2] = round_bf16(hi.x) | (static_cast<uint32_t>(round_bf16(hi.y)) << 16);
    xw[c][3] = round_bf16(hi.z) | (static_cast<uint32_t>(round_bf16(hi.w)) << 16);
    const uint32_t rw[4] = {rv[c].x, rv[c].y, rv[c].z, rv[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = bf16_to_f32(static_cast<uint16_t>(xw[c][e])) + bf16_to_f32(static_cast<uint16_t>(rw[e]));
      const float a1 = bf16_to_f32(static_cast<uint16_t>(xw[c][e] >> 16)) + bf16_to_f32(static_cast<uint16_t>(rw[e] >> 16));
      xw[c][e] = round_bf16(a0) | (static_cast<uint32_t>(round_bf16(a1)) << 16);
    }
    if (i < H) {
      *reinterpret_cast<uint4*>(rr + i) = make_uint4(xw[c][0], xw[c][1], xw[c][2], xw[c][3]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = bf16_to_f32(static_cast<uint16_t>(xw[c][e]));
        const float a1 = bf16_to_f32(static_cast<uint16_t>(xw[c][e] >> 16));
        ss += a0 * a0 + a1 * a1;
      }
    }
  }
  const float rs = rsqrtf(block_sum_f32(ss, sh) / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int i = (c * kThreads + threadIdx.x) * 8;
    if (i >= H) continue;
    const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float n0 = bf16_to_f32(round_bf16(bf16_to_f32(static_cast<uint16_t>(xw[c][e])) * rs));
      const float n1 = bf16_to_f32(round_bf16(bf16_to_f32(static_cast<uint16_t>(xw[c][e] >> 16)) * rs));
      const float y0 = bf16_to_f32(static_cast<uint16_t>(ww[e])) * n0;
      const float y1 = bf16_to_f32(static_cast<uint16_t>(ww[e] >> 16)) * n1;
      ow[e] = round_bf16(y0) | (static_cast<uint32_t>(round_bf16(y1)) << 16);
    }
    *reinterpret_cast<uint4*>(out + row * H + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

template <int CPT>
bool launch_rms_part(int kb, dim3 grid, hipStream_t s, uint16_t* rp, const uint16_t* wp,
                     uint16_t* op, int hidden, float eps, const float* part, int ks,
                     int64_t slice) {
  // at most 32 float4 of partials in registers per thread
  switch (kb) {
    case 1: hipLaunchKernelGGL((rms_norm_part_kernel<CPT, 1>), grid, dim3(kThreads), 0, s, rp, wp, op, hidden, eps, part, ks, slice); return true;
    case 2: hipLaunchKernelGGL((rms_norm_part_kernel<CPT, 2>), grid, dim3(kThreads), 0, s, rp, wp, op, hidden, eps, part, ks, slice); return true;
    case 4: hipLaunchKernelGGL((rms_norm_part_kernel<CPT, 4>), grid, dim3(kThreads), 0, s, rp, wp, op, hidden, eps, part, ks, slice); return true;
    case 8:
      if constexpr (CPT <= 2) {
        hipLaunchKernelGGL((rms_norm_part_kernel<CPT, 8>), grid, dim3(kThreads), 0, s, rp, wp, op, hidden, eps, part, ks, slice);
        return true;
      }
      return false;
    case 16:
      if constexpr (CPT <= 1) {
        hipLaunchKernelGGL((rms_norm_part_kernel<CPT, 16>), grid, dim3(kThreads), 0, s, rp, wp, op, hidden, eps, part, ks, slice);
        return true;
      }
      return false;
    default:
      return false;
  }
}

// In-place neox rotary embedding of q [T, Hq, D] and k [T, Hkv, D]: for i < D/2,
// (x_i, x_{i+D/2}) -> (x_i c - x_{i+D/2} s, x_{i+D/2} c + x_i s) with c, s = cos/sin[pos][i]
// from bf16 tables [max_pos, D] (engine/model.py:92-94, 120-124).  One thread per pair.
__global__ __launch_bounds__(kThreads) void rope_kernel(uint16_t* __restrict__ q, int64_t q_ts,
                                                        int64_t q_hs, uint16_t* __restrict__ k,
                                                        int64_t k_ts, int64_t k_hs,
                                                        const int64_t* __restrict__ pos,
                                                        const uint16_t* __restrict__ cos,
                                                        const uint16_t* __restrict__ sin,
                                                        int64_t tab_stride, int T, int Hq, int Hkv,
                                                        int D, int max_pos) {
  const int half = D / 2;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t per_tok = static_cast<int64_t>(Hq + Hkv) * half;
  if (gid >= per_tok * T) return;
  const int t = static_cast<int>(gid / per_tok);
  const int rem = static_cast<int>(gid % per_tok);
  const int h = rem / half, i = rem % half;
  uint16_t* base = h < Hq ? q + t * q_ts + h * q_hs : k + t * k_ts + (h - Hq) * k_hs;
  int64_t p = pos[t];
  p = p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p);
  const float c = bf16_to_f32(cos[p * tab_stride + i]);
  const float s = bf16_to_f32(sin[p * tab_stride + i]);
  const float x1 = bf16_to_f32(base[i]), x2 = bf16_to_f32(base[i + half]);
  // explicit fma forms, shared with the fused qkv epilogue (one rounding of x1 c - x2 s via
  // fma(x1, c, -(x2 s)), and of x2 c + x1 s via fma(x2, c, x1 s))
  base[i] = round_bf16(fmaf(x1, c, -(x2 * s)));
  base[i + half] = round_bf16(fmaf(x2, c, x1 * s));
}

__device__ __forceinline__ uint32_t pack_sum_bf16(float a, float b) {
  return round_bf16(a) | (static_cast<uint32_t>(round_bf16(b)) << 16);
}

// out[t, j] = silu(gu[t, j]) * gu[t, F + j] (engine/model.py:250-253), 8 elements per thread.
// With `part` set, gu is not read: gu[t] = bf16(sum of the ks fp32 slices part[k * slice +
// t * 2F]), the split-K partials of the gate_up projection, reduced in its own order.
// KS > 0: partials with the slice count bounded at compile time, all 4 * KS loads issued
// before the first add (one global round trip); KS = 0: the runtime-bounded path.
template <int KS>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                            uint16_t* __restrict__ out, int64_t T,
                                                            int F, const float* __restrict__ part,
                                                            int ks, int64_t slice) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int per_row = F / 8;
  if (gid >= T * per_row) return;
  const int64_t t = gid / per_row;
  const int j = static_cast<int>(gid % per_row) * 8;
  uint32_t gw[4], uw[4];
  if (part) {
    const float* pg = part + t * 2 * F + j;
    float4 g0, g1, u0, u1;
    if constexpr (KS > 0) {
      Partials4<KS> pg0, pg1, pu0, pu1;
      pg0.load(pg, ks, slice);
      pg1.load(pg + 4, ks, slice);
      pu0.load(pg + F, ks, slice);
      pu1.load(pg + F + 4, ks, slice);
      g0 = pg0.sum(ks); g1 = pg1.sum(ks); u0 = pu0.sum(ks); u1 = pu1.sum(ks);
    } else {
      g0 = sum_partials4(pg, ks, slice); g1 = sum_partials4(pg + 4, ks, slice);
      u0 = sum_partials4(pg + F, ks, slice); u1 = sum_partials4(pg + F + 4, ks, slice);
    }
    gw[0] = pack_sum_bf16(g0.x, g0.y); gw[1] = pack_sum_bf16(g0.z, g0.w);
    gw[2] = pack_sum_bf16(g1.x, g1.y); gw[3] = pack_sum_bf16(g1.z, g1.w);
    uw[0] = pack_sum_bf16(u0.x, u0.y); uw[1] = pack_sum_bf16(u0.z, u0.w);
    uw[2] = pack_sum_bf16(u1.x, u1.y); uw[3] = pack_sum_bf16(u1.z, u1.w);
  } else {
    const uint4 gv = *reinterpret_cast<const uint4*>(gu + t * 2 * F + j);
    const uint4 uv = *reinterpret_cast<const uint4*>(gu + t * 2 * F + F + j);
    gw[0] = gv.x; gw[1] = gv.y; gw[2] = gv.z; gw[3] = gv.w;
    uw[0] = uv.x; uw[1] = uv.y; uw[2] = uv.z; uw[3] = uv.w;
  }
  uint32_t ow[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float r[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const float g = bf16_to_f32(static_cast<uint16_t>(gw[e] >> (16 * hh)));
      const float u = bf16_to_f32(static_cast<uint16_t>(uw[e] >> (16 * hh)));
      r[hh] = g / (1.0f + __expf(-g)) * u;
    }
    ow[e] = round_bf16(r[0]) | (static_cast<uint32_t>(round_bf16(r[1])) << 16);
  }
  *reinterpret_cast<uint4*>(out + t * F + j) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

}  // namespace

extern "C" int coopt_rms_norm(const void* x, void* residual, const void* weight, void* out,
                              int64_t rows, int hidden, float eps, coopt_stream_t stream) {
  COOPT_REQUIRE(rows >= 0 && hidden > 0 && hidden % 8 == 0, "hidden must be a multiple of 8");
  if (rows == 0) return COOPT_OK;
  COOPT_REQUIRE(x && weight && out, "null pointer");
  COOPT_REQUIRE(coopt::aligned16(x) && coopt::aligned16(weight) && coopt::aligned16(out) &&
                    (residual == nullptr || coopt::aligned16(residual)),
                "rows must be 16-byte aligned");
  coopt::clear_error();
  const dim3 grid(static_cast<unsigned>(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  uint16_t* rp = static_cast<uint16_t*>(residual);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  uint16_t* op = static_cast<uint16_t*>(out);
  const int cpt = (hidden + kThreads * 8 - 1) / (kThreads * 8);
  switch (cpt) {
    case 1: hipLaunchKernelGGL(rms_norm_reg_kernel<1>, grid, dim3(kThreads), 0, s, xp, rp, wp, op, hidden, eps, nullptr, 0, 0); break;
    case 2: hipLaunchKernelGGL(rms_norm_reg_kernel<2>, grid, dim3(kThreads), 0, s, xp, rp, wp, op, hidden, eps, nullptr, 0, 0); break;
    case 3: hipLaunchKernelGGL(rms_norm_reg_kernel<3>, grid, dim3(kThreads), 0, s, xp, rp, wp, op, hidden, eps, nullptr, 0, 0); break;
    case 4: hipLaunchKernelGGL(rms_norm_reg_kernel<4>, grid, dim3(kThreads), 0, s, xp, rp, wp, op, hidden, eps, nullptr, 0, 0); break;
    default: hipLaunchKernelGGL(rms_norm_kernel, grid, dim3(kThreads), 0, s, xp, rp, wp, op, hidden, eps);
  }
  return coopt::check_launch("coopt_rms_norm");
}

extern "C" int coopt_rms_norm_partials(const float* part, int ks, int64_t slice_stride,
                                       void* residual, const void* weight, void* out,
                                       int64_t rows, int hidden, float eps,
                                       coopt_stream_t stream) {
  COOPT_REQUIRE(rows >= 0 && hidden > 0 && hidden % 8 == 0 && hidden <= kThreads * 8 * 4,
                "hidden must be a multiple of 8, at most 8192");
  COOPT_REQUIRE(ks >= 1 && ks <= 16, "1 to 16 partial slices");
  COOPT_REQUIRE(slice_stride >= rows * hidden && slice_stride % 4 == 0, "bad slice stride");
  if (rows == 0) return COOPT_OK;
  COOPT_REQUIRE(part && weight && out, "null pointer");
  COOPT_REQUIRE(coopt::aligned16(part) && coopt::aligned16(weight) && coopt::aligned16(out) &&
                    (residual == nullptr || coopt::aligned16(residual)),
                "rows must be 16-byte aligned");
  coopt::clear_error();
  const dim3 grid(static_cast<unsigned>(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* rp = static_cast<uint16_t*>(residual);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  uint16_t* op = static_cast<uint16_t*>(out);
  const int cpt = (hidden + kThreads * 8 - 1) / (kThreads * 8);
  if (rp != nullptr) {
    const int kb = partials_bound(ks);
    bool done = false;
    switch (cpt) {
      case 1: done = launch_rms_part<1>(kb, grid, s, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
      case 2: done = launch_rms_part<2>(kb, grid, s, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
      case 3: done = launch_rms_part<3>(kb, grid, s, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
      case 4: done = launch_rms_part<4>(kb, grid, s, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
    }
    if (done) return coopt::check_launch("coopt_rms_norm_partials");
  }
  switch (cpt) {
    case 1: hipLaunchKernelGGL(rms_norm_reg_kernel<1>, grid, dim3(kThreads), 0, s, nullptr, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
    case 2: hipLaunchKernelGGL(rms_norm_reg_kernel<2>, grid, dim3(kThreads), 0, s, nullptr, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
    case 3: hipLaunchKernelGGL(rms_norm_reg_kernel<3>, grid, dim3(kThreads), 0, s, nullptr, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
    default: hipLaunchKernelGGL(rms_norm_reg_kernel<4>, grid, dim3(kThreads), 0, s, nullptr, rp, wp, op, hidden, eps, part, ks, slice_stride); break;
  }
  return coopt::check_launch("coopt_rms_norm_partials");
}

extern "C" int coopt_rope(void* q, int64_t q_tok_stride, int64_t q_head_stride, void* k,
                          int64_t k_tok_stride, int64_t k_head_stride, const int64_t* positions,
                          const void* cos, const void* sin, int64_t table_stride, int max_pos,
                          int T, int Hq, int Hkv, int D, coopt_stream_t stream) {
  COOPT_REQUIRE(T >= 0 && Hq > 0 && Hkv >= 0 && D > 0 && D % 2 == 0 && max_pos > 0, "bad sizes");
  if (T == 0) return COOPT_OK;
  COOPT_REQUIRE(q && positions && cos && sin && (k || Hkv == 0), "null pointer");
  coopt::clear_error();
  const int64_t total = static_cast<int64_t>(T) * (Hq + Hkv) * (D / 2);
  hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint16_t*>(q), q_tok_stride, q_head_stride,
                     static_cast<uint16_t*>(k), k_tok_stride, k_head_stride, positions,
                     static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin),
                     table_stride, T, Hq, Hkv, D, max_pos);
  return coopt::check_launch("coopt_rope");
}

extern "C" int coopt_silu_mul(const void* gate_up, void* out, int64_t T, int F,
                              coopt_stream_t stream) {
  COOPT_REQUIRE(T >= 0 && F > 0 && F % 8 == 0, "F must be a multiple of 8");
  if (T == 0) return COOPT_OK;
  COOPT_REQUIRE(gate_up && out && coopt::aligned16(gate_up) && coopt::aligned16(out),
                "null or misaligned pointer");
  coopt::clear_error();
  const int64_t total = T * (F / 8);
  hipLaunchKernelGGL(silu_mul_kernel<0>, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), T, F,
                     nullptr, 0, 0);
  return coopt::check_launch("coopt_silu_mul");
}

extern "C" int coopt_silu_mul_partials(const float* part, int ks, int64_t slice_stride, void* out,
                                       int64_t T, int F, coopt_stream_t stream) {
  COOPT_REQUIRE(T >= 0 && F > 0 && F % 8 == 0, "F must be a multiple of 8");
  COOPT_REQUIRE(ks >= 1 && ks <= 16, "1 to 16 partial slices");
  COOPT_REQUIRE(slice_stride >= T * 2 * F && slice_stride % 4 == 0, "bad slice stride");
  if (T == 0) return COOPT_OK;
  COOPT_REQUIRE(part && out && coopt::aligned16(part) && coopt::aligned16(out),
                "null or misaligned pointer");
  coopt::clear_error();
  const int64_t total = T * (F / 8);
  const dim3 grid(static_cast<unsigned>((total + kThreads - 1) / kThreads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* op = static_cast<uint16_t*>(out);
  switch (partials_bound(ks)) {  // at most 32 float4 of partials in registers per thread
    case 1: hipLaunchKernelGGL(silu_mul_kernel<1>, grid, dim3(kThreads), 0, st, nullptr, op, T, F, part, ks, slice_stride); break;
    case 2: hipLaunchKernelGGL(silu_mul_kernel<2>, grid, dim3(kThreads), 0, st, nullptr, op, T, F, part, ks, slice_stride); break;
    case 4: hipLaunchKernelGGL(silu_mul_kernel<4>, grid, dim3(kThreads), 0, st, nullptr, op, T, F, part, ks, slice_stride); break;
    case 8: hipLaunchKernelGGL(silu_mul_kernel<8>, grid, dim3(kThreads), 0, st, nullptr, op, T, F, part, ks, slice_stride); break;
    default: hipLaunchKernelGGL(silu_mul_kernel<0>, grid, dim3(kThreads), 0, st, nullptr, op, T, F, part, ks, slice_stride); break;
  }
  return coopt::check_launch("coopt_silu_mul_partials");
}
