// Device bookkeeping of one speculative step for the batch in slots [0, Bc) of the decoder's
// state (engine/engine.py:338-470, for a batch in which every sequence decodes).  The
// reference keeps this state in Python lists and walks them on the host between launches;
// here it stays on the GPU and three single-workgroup launches do the walking, so a whole
// step can be replayed from one HIP graph:
//
//   begin          before the draft: the step's row of the uniform table, each sequence's
//                  mode (speculate when gamma > 0 and lag <= 2, catch up when lagging,
//                  plain decode when gamma = 0; engine/engine.py:354-372), the draft
//                  catch-up's rows and tokens, the row of the catch-up whose logits the
//                  first proposal is drawn from, the start row and the real-row count of
//                  every later proposal (draft_computed advancing by one per active
//                  proposal, :380-389), the verify rows [last token] + drafts (:414-417)
//                  and draft_computed after the draft phase;
//   verify_tokens  after the proposals: the drafted tokens into the verify rows and into
//                  the accept test's [Bc, S_t - 1] token rows;
//   commit         after the accept: the kept tokens appended to the history (:455),
//                  num_computed = len - 1 and draft_computed clamped to it (the rollback of
//                  :463-470, stored as the length update), and the emitted / drafted /
//                  accepted counters (:444-446).
//
// Everything here is a function of the state and the kernels' own outputs, so graph replays
// and eager steps are identical.  Sizes are a few hundred sequences: one workgroup, a thread
// per sequence.
#include "common.h"

namespace {

constexpr int kThreads = 256;

struct BeginArgs {
  const float* u_table;
  int64_t u_rows;
  int nu;
  int64_t* u_counter;
  float* u;
  const uint8_t* live;
  const int64_t* gamma;
  const int64_t* n;
  const int64_t* dc;
  const int64_t* hist;
  int64_t hist_stride;
  int64_t max_len;
  int Bc, G, S_c, S_t;
  int32_t* gamma_eff;
  int64_t* cu_start;
  int64_t* cu_nreal;
  int64_t* cu_tokens;
  int64_t* cu_keep_rows;
  int64_t* pr_start;
  int64_t* pr_nreal;
  int64_t pr_stride;
  int64_t* v_start;
  int64_t* v_nreal;
  int32_t* v_tokens;
  int64_t* dc_final;
};

__global__ __launch_bounds__(kThreads) void step_begin_kernel(BeginArgs a) {
  __shared__ int64_t sh_row, sh_ctr;
  const int tid = threadIdx.x;
  if (tid == 0) {
    const int64_t c = *a.u_counter;
    int64_t r = c % a.u_rows;
    if (r < 0) r += a.u_rows;
    sh_ctr = c;
    sh_row = r;
  }
  __syncthreads();
  const float* urow = a.u_table + sh_row * a.nu;
  for (int k = tid; k < a.nu; k += kThreads) a.u[k] = urow[k];
  if (tid == 0) *a.u_counter = sh_ctr + 1;

  const int64_t last = a.max_len - 1;
  for (int b = tid; b < a.Bc; b += kThreads) {
    const bool lv = a.live[b] != 0;
    const int64_t gq = a.gamma[b], nn = a.n[b], d = a.dc[b];
    const int64_t lag = nn - d;
    const bool want = lv && gq > 0;
    const bool spec = want && lag <= 2;
    const bool lagging = want && lag > 2;
    const int64_t ge = spec ? gq : 0;
    // catch-up rows: the whole lag when speculating, min(lag - 1, S_c) when lagging
    const int64_t m = spec ? lag : (lagging ? min(lag - 1, static_cast<int64_t>(a.S_c)) : 0);
    a.gamma_eff[b] = static_cast<int32_t>(ge);
    const int64_t* h = a.hist + static_cast<int64_t>(b) * a.hist_stride;
    int64_t dc1 = d;
    if (a.G > 0) {
      const int64_t st = lv ? d : 0;
      a.cu_start[b] = st;
      a.cu_nreal[b] = m;
      for (int j = 0; j < a.S_c; ++j)
        a.cu_tokens[static_cast<int64_t>(b) * a.S_c + j] = h[min(st + j, last)];
      a.cu_keep_rows[b] = static_cast<int64_t>(b) * a.S_c + max(m - 1, static_cast<int64_t>(0));
      dc1 = d + m;
      for (int i = 1; i < a.G; ++i) {
        const int64_t act = (spec && ge > i) ? 1 : 0;
        a.pr_start[(i - 1) * a.pr_stride + b] = lv ? dc1 : 0;
        a.pr_nreal[(i - 1) * a.pr_stride + b] = act;
        dc1 += act;
      }
    }
    const int64_t vs = lv ? nn - 1 : 0;
    a.v_start[b] = vs;
    a.v_nreal[b] = lv ? ge + 1 : 0;
    a.v_tokens[static_cast<int64_t>(b) * a.S_t] = static_cast<int32_t>(h[min(max(vs, static_cast<int64_t>(0)), last)]);
    a.dc_final[b] = dc1;
  }
}

// proposals [G][prop_stride] (proposal i of sequence b at i * prop_stride + b) -> verify rows
// [b][1 + i] of v_tokens [Bc][S_t] and the accept's draft rows [b][i] of draft_tokens
// [Bc][S_t - 1]
__global__ __launch_bounds__(kThreads) void verify_tokens_kernel(const int32_t* __restrict__ prop,
                                                                 int64_t prop_stride, int Bc, int S_t,
                                                                 int32_t* __restrict__ v_tokens,
                                                                 int32_t* __restrict__ draft_tokens) {
  const int g = S_t - 1;
  const int total = Bc * g;
  for (int idx = threadIdx.x; idx < total; idx += kThreads) {
    const int b = idx / g, i = idx - b * g;
    const int32_t t = prop[static_cast<int64_t>(i) * prop_stride + b];
    v_tokens[static_cast<int64_t>(b) * S_t + 1 + i] = t;
    draft_tokens[idx] = t;
  }
}

__device__ __forceinline__ int64_t block_sum(int64_t v, int64_t* sh) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((tid & 63) == 0) sh[tid >> 6] = v;
  __syncthreads();
  int64_t s = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) s += sh[w];
  return s;
}

__global__ __launch_bounds__(kThreads) void step_commit_kernel(
    const uint8_t* __restrict__ live, const int32_t* __restrict__ acc_len,
    const int32_t* __restrict__ tokens, int S_t, const int32_t* __restrict__ gamma_eff,
    const int64_t* __restrict__ dc_final, int64_t* __restrict__ n, int64_t* __restrict__ dc,
    int64_t* __restrict__ hist, int64_t hist_stride, int64_t max_len, int64_t* emitted,
    int64_t* drafted, int64_t* accepted, int Bc) {
  __shared__ int64_t sh[3][kThreads / 64];
  int64_t e = 0, dr = 0, ac = 0;
  for (int b = threadIdx.x; b < Bc; b += kThreads) {
    const bool lv = live[b] != 0;
    const int64_t k = lv ? min(max(acc_len[b], 0), S_t - 1) : 0;
    const int64_t nn = n[b];
    if (lv) {
      int64_t* h = hist + static_cast<int64_t>(b) * hist_stride;
      for (int64_t j = 0; j <= k; ++j)
        if (nn + j < max_len) h[nn + j] = tokens[static_cast<int64_t>(b) * S_t + j];
      const int64_t new_n = nn + k + 1;
      n[b] = new_n;
      dc[b] = min(dc_final[b], new_n - 1);
      e += k + 1;
    }
    dr += gamma_eff[b];
    ac += k;
  }
  e = block_sum(e, sh[0]);
  dr = block_sum(dr, sh[1]);
  ac = block_sum(ac, sh[2]);
  if (threadIdx.x == 0) {
    *emitted += e;
    *drafted += dr;
    *accepted += ac;
  }
}

}  // namespace

extern "C" int coopt_spec_step_begin(
    const float* u_table, int64_t u_rows, int nu, int64_t* u_counter, float* u,
    const uint8_t* live, const int64_t* gamma, const int64_t* n, const int64_t* dc,
    const int64_t* hist, int64_t hist_stride, int64_t max_len, int Bc, int G, int S_c, int S_t,
    int32_t* gamma_eff, int64_t* cu_start, int64_t* cu_nreal, int64_t* cu_tokens,
    int64_t* cu_keep_rows, int64_t* pr_start, int64_t* pr_nreal, int64_t pr_stride,
    int64_t* v_start, int64_t* v_nreal, int32_t* v_tokens, int64_t* dc_final,
    coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(Bc >= 0 && G >= 0 && S_t >= 1 && nu >= 0, "negative size or S_t < 1");
  COOPT_REQUIRE(u_rows >= 1 && max_len >= 1 && hist_stride >= max_len,
                "u_rows, max_len must be positive and hist_stride >= max_len");
  COOPT_REQUIRE(u_table && u_counter && (u || nu == 0), "null pointer (uniforms)");
  if (Bc > 0) {
    COOPT_REQUIRE(live && gamma && n && dc && hist && gamma_eff && v_start && v_nreal &&
                      v_tokens && dc_final, "null pointer");
    if (G > 0) {
      COOPT_REQUIRE(S_c >= 1, "S_c must be >= 1 when the draft runs");
      COOPT_REQUIRE(cu_start && cu_nreal && cu_tokens && cu_keep_rows, "null pointer (catch-up)");
    }
    if (G > 1) {
      COOPT_REQUIRE(pr_start && pr_nreal && pr_stride >= Bc, "null pointer or pr_stride < Bc");
    }
  }
  BeginArgs a{u_table, u_rows, nu, u_counter, u, live, gamma, n, dc, hist, hist_stride, max_len,
              Bc, G, S_c, S_t, gamma_eff, cu_start, cu_nreal, cu_tokens, cu_keep_rows, pr_start,
              pr_nreal, pr_stride, v_start, v_nreal, v_tokens, dc_final};
  hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return coopt::check_launch("coopt_spec_step_begin");
}

extern "C" int coopt_spec_step_verify_tokens(const int32_t* proposals, int64_t prop_stride, int Bc,
                                             int S_t, int32_t* v_tokens, int32_t* draft_tokens,
                                             coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(Bc >= 0 && S_t >= 1, "negative size or S_t < 1");
  if (Bc == 0 || S_t == 1) return COOPT_OK;
  COOPT_REQUIRE(proposals && v_tokens && draft_tokens, "null pointer");
  COOPT_REQUIRE(prop_stride >= Bc, "prop_stride < Bc");
  hipLaunchKernelGGL(verify_tokens_kernel, dim3(1), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), proposals, prop_stride, Bc, S_t,
                     v_tokens, draft_tokens);
  return coopt::check_launch("coopt_spec_step_verify_tokens");
}

extern "C" int coopt_spec_step_commit(const uint8_t* live, const int32_t* accepted_len,
                                      const int32_t* tokens, int S_t, const int32_t* gamma_eff,
                                      const int64_t* dc_final, int64_t* n, int64_t* dc,
                                      int64_t* hist, int64_t hist_stride, int64_t max_len,
                                      int64_t* emitted, int64_t* drafted, int64_t* accepted, int Bc,
                                      coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(Bc >= 0 && S_t >= 1, "negative size or S_t < 1");
  COOPT_REQUIRE(max_len >= 1 && hist_stride >= max_len, "max_len >= 1 and hist_stride >= max_len");
  COOPT_REQUIRE(emitted && drafted && accepted, "null pointer (counters)");
  if (Bc > 0) {
    COOPT_REQUIRE(live && accepted_len && tokens && gamma_eff && dc_final && n && dc && hist,
                  "null pointer");
  }
  hipLaunchKernelGGL(step_commit_kernel, dim3(1), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), live, accepted_len, tokens, S_t,
                     gamma_eff, dc_final, n, dc, hist, hist_stride, max_len, emitted, drafted,
                     accepted, Bc);
  return coopt::check_launch("coopt_spec_step_commit");
}
