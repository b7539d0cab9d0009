/*
 * coopt_amd.h -- C ABI of libcoopt_amd.so, the MI355X (gfx950) kernels behind the
 * speculative verify/accept path and the paged KV cache it reads.
 *
 * Conventions shared by every entry point:
 *   - Plain pointers to device memory, element strides (not bytes), int sizes.
 *     The last dimension of every tensor argument (head_dim, vocab) is contiguous.
 *   - Every call is enqueued on `stream` (a hipStream_t; NULL = the null stream),
 *     allocates nothing, never synchronises the host, and is safe to record into a
 *     HIP graph. Calls are reentrant; the only global is the per-thread error text.
 *   - Return value: COOPT_OK (0) or a negative COOPT_E* code; coopt_last_error()
 *     then holds a message for the calling thread.
 *   - Workspaces are caller-owned device buffers of at least the size the matching
 *     *_workspace() function returns.  They need no initialisation and carry nothing from
 *     one call to the next; kernels exchange partial results through them only across
 *     launch boundaries (no cross-workgroup fences or counters).  One workspace serves calls
 *     of any shape, one call at a time: two calls that overlap in time on it race.
 *
 * Reference interfaces replaced (paths under mohsinmubarak/iitj-llm-coopt):
 *   coopt_kv_write          vLLM reshape_and_cache_flash   engine/model.py:242-243
 *                           (semantics: engine/model.py:190,201-203; tests/kv_write_check.py:26-30)
 *   coopt_verify_attention  vLLM flash_attn_varlen_func    engine/model.py:244-247 (and :204-207)
 *   coopt_accept_sample     spec_decode.verify / sample     engine/spec_decode.py:12-49,
 *                           batched as at engine/engine.py:421-446
 *   coopt_quantize /        kv_tier_manager.quantize /     engine/kv_tier_manager.py:21-41
 *   coopt_dequantize        dequantize
 *   coopt_kv_swap_out /     quantize(cache[blocks], bits) / engine/kv_tier_manager.py:93-101
 *   coopt_kv_swap_in        cache[blocks] = dequantize(..)  engine/kv_tier_manager.py:113-119
 *   coopt_kv_swap_*_caches  the same over every layer's K   engine/kv_tier_manager.py:93-101,
 *                           and V cache in one launch       113-119 (the per-layer loops)
 *   coopt_qkv_epilogue      split + rotary_embedding +      engine/model.py:238-243
 *                           reshape_and_cache_flash
 *   coopt_kv_copy_blocks    buf[dst].copy_(buf[src]) per    engine/elastic.py:131 via
 *                           migrated block                  engine/block_manager.py:165-187
 *   coopt_softmax           torch.softmax(logits / T)       engine/spec_decode.py:16
 *   coopt_sample_probs      the same, for rows just sampled engine/spec_decode.py:16
 *   coopt_sample            spec_decode.sample (tokens      engine/spec_decode.py:12-17
 *                           and probabilities) at T > 0
 *   coopt_rms_norm          vLLM rms_norm / fused_add_rms_norm  engine/model.py:234, 236, 249, 254
 *   coopt_rope              vLLM rotary_embedding (neox)    engine/model.py:239
 *   coopt_silu_mul          vLLM silu_and_mul               engine/model.py:251-252
 *   coopt_row_slots         slot_mapping / positions /      engine/block_manager.py:216-220,
 *                           seq_lens of a padded row batch  engine/batch.py:23-55
 *   coopt_linear            F.linear projections at decode  engine/model.py:238, 248, 250,
 *                           / verify row counts             253 (qkv, o, gate_up, down)
 *   coopt_linear_*packed    the same, tile-packed weights   engine/model.py:238, 248, 253
 *   coopt_linear_silu_packed  gate_up + silu_and_mul        engine/model.py:250-252
 *   coopt_spec_step_begin /  the host-side bookkeeping of   engine/engine.py:354-389,
 *   _verify_tokens / _commit one speculative step: lag,     414-417, 444-446, 455,
 *                           catch-up, proposal rows, verify 463-470
 *                           rows, append, rollback, counters
 */
#ifndef COOPT_AMD_H
#define COOPT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* coopt_stream_t; /* hipStream_t */

enum {
  COOPT_OK = 0,
  COOPT_EINVAL = -1,     /* bad argument (null pointer, unsupported shape, misalignment) */
  COOPT_EHIP = -2,       /* the HIP runtime reported an error (launch failure) */
  COOPT_EWORKSPACE = -3  /* workspace smaller than the *_workspace() size */
};

enum {
  COOPT_DT_F32 = 0,
  COOPT_DT_BF16 = 1,
  COOPT_DT_F16 = 2,
  COOPT_DT_I8 = 3
};

/* Message describing the last failed call on this thread ("" if none). */
const char* coopt_last_error(void);

/* hipRuntimeGetVersion() of the HIP runtime this library is bound to. */
int coopt_hip_runtime_version(int* version);

/*
 * Paged KV write.  Replaces reshape_and_cache_flash(k, v, k_cache, v_cache, slot_mapping,
 * "auto", k_scale, v_scale) at engine/model.py:242-243; the reference defines it as
 *   k_cache[slot // block_size, slot % block_size] = k   (engine/model.py:190, 201-203).
 *
 *   k, v        [T, Hkv, D] bf16 with strides (k_tok, k_head, 1) and (v_tok, v_head, 1)
 *   cache_dtype COOPT_DT_BF16: k_cache/v_cache are bf16 [NB, block_size, Hkv, D]
 *               COOPT_DT_I8:   k_cache/v_cache are int8 codes of the same shape and
 *                              k_scale/v_scale are fp16 [NB, block_size, Hkv]; each (token, head)
 *                              vector is quantised as kv_tier_manager.quantize(x, 8) does
 *                              (engine/kv_tier_manager.py:21-31), codes and scales bit-exact.
 *   cache strides (c_blk, c_tok, c_head, 1) may describe a strided per-layer view of a
 *   block-major buffer (engine/elastic.py:74-77); scale strides (s_blk, s_tok, s_head).
 *   slot_mapping [T] int64.  A slot < 0 or >= num_blocks * block_size is skipped (padding).
 *   D must be a multiple of 8 with D/8 a power of two <= 64; k/v/cache rows 16-byte aligned.
 */
int coopt_kv_write(int cache_dtype,
                   const void* k, const void* v, int64_t k_tok_stride, int64_t k_head_stride,
                   int64_t v_tok_stride, int64_t v_head_stride, void* k_cache, void* v_cache,
                   int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                   void* k_scale, void* v_scale,
                   int64_t s_blk_stride, int64_t s_tok_stride, int64_t s_head_stride,
                   const int64_t* slot_mapping, int T, int Hkv, int D, int block_size,
                   int64_t num_blocks, coopt_stream_t stream);

/*
 * The step after the qkv projection in one launch: split q/k/v, neox RoPE on q and k, q to
 * q_out, k and v into the paged cache -- the chain  q, k, v = F.linear(h, qkv).split(...);
 * rotary_embedding(positions, q, k, ...); reshape_and_cache_flash(k, v, ...)  at
 * engine/model.py:238-243.
 *   input: either qkv [T, (Hq + 2 Hkv) D] bf16 (row stride qkv_tok_stride, part NULL), or
 *          part: the projection's fp32 split-K partials (coopt_linear_partials: ks slices of
 *          slice_stride floats, rows (Hq + 2 Hkv) D wide), reduced in coopt_linear's order
 *          and rounded to bf16 first (qkv NULL).
 *   RoPE: as coopt_rope (cos/sin bf16 [max_pos, table_stride], positions clamped).
 *   q_out [T, Hq, D] bf16 (strides q_tok_stride, q_head_stride); the cache arguments are
 *   those of coopt_kv_write, including slot < 0 for rows that write no entry.
 *   D in {64, 128, 256}.  Results equal coopt_linear + coopt_rope + coopt_kv_write bit for bit.
 */
int coopt_qkv_epilogue(int cache_dtype, const void* qkv, int64_t qkv_tok_stride,
                       const float* part, int ks, int64_t slice_stride,
                       const int64_t* positions, const void* cos, const void* sin,
                       int64_t table_stride, int max_pos, void* q_out, int64_t q_tok_stride,
                       int64_t q_head_stride, void* k_cache, void* v_cache,
                       int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                       void* k_scale, void* v_scale, int64_t s_blk_stride,
                       int64_t s_tok_stride, int64_t s_head_stride,
                       const int64_t* slot_mapping, int T, int Hq, int Hkv, int D,
                       int block_size, int64_t num_blocks, coopt_stream_t stream);

/*
 * Symmetric absmax codec over contiguous rows, kv_tier_manager.quantize / dequantize
 * (engine/kv_tier_manager.py:21-41).
 *   coopt_quantize:   x [rows, D] (in_dtype BF16/F16/F32) -> q, scale [rows] fp16.
 *                     bits 8: q int8 [rows, D];  bits 4: q uint8 [rows, D/2], even element in
 *                     the low nibble, odd element in the high nibble, both offset by +8.
 *   coopt_dequantize: q, scale -> out [rows, D] in out_dtype (BF16/F16/F32).
 * D must be even and <= 4096.
 */
int coopt_quantize(int bits, int in_dtype, const void* x, int64_t rows, int D,
                   void* q, void* scale, coopt_stream_t stream);
int coopt_dequantize(int bits, const void* q, const void* scale, int64_t rows, int D,
                     int out_dtype, void* out, coopt_stream_t stream);

/*
 * KV tier swap codec, one launch per (layer, K or V) cache.  Replaces the per-layer
 *   q, s = quantize(cache[blocks], bits)            (swap_out, engine/kv_tier_manager.py:99)
 *   cache[blocks] = dequantize(q, s, bits, dtype)   (swap_in, engine/kv_tier_manager.py:119)
 * with the gather / scatter fused into the codec.
 *   cache        [num_blocks, block_size, Hkv, D] with strides (c_blk, c_tok, c_head, 1):
 *                COOPT_DT_BF16 values, or COOPT_DT_I8 codes with fp16 cache_scale
 *                [num_blocks, block_size, Hkv] (strides s_blk, s_tok, s_head).
 *   block_ids    [num_ids] int64 device array; q / scale are contiguous
 *                [num_ids, block_size, Hkv, D'] and [num_ids, block_size, Hkv] (fp16):
 *                bits 16: q holds bf16 copies (D' = D, no scale); bits 8: int8 codes (D' = D);
 *                bits 4: two codes per byte (D' = D/2), even element in the low nibble, +8.
 *   Codes and scales are those of kv_tier_manager.quantize on the GPU (bit-exact); swap_in
 *   writes bf16(float(code) * float(scale)).  An INT8 cache (bits must be 8) is copied code for
 *   code with its scales, both ways (lossless).  Ids outside [0, num_blocks) are read as zero
 *   vectors by swap_out and skipped by swap_in.  D must be 8 * a power of two, <= 512.
 */
int coopt_kv_swap_out(int bits, int cache_dtype, const void* cache,
                      int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                      const void* cache_scale, int64_t s_blk_stride, int64_t s_tok_stride,
                      int64_t s_head_stride, const int64_t* block_ids, int num_ids,
                      int block_size, int Hkv, int D, int64_t num_blocks, void* q, void* scale,
                      coopt_stream_t stream);
int coopt_kv_swap_in(int bits, int cache_dtype, const void* q, const void* scale,
                     const int64_t* block_ids, int num_ids, int block_size, int Hkv, int D,
                     int64_t num_blocks, void* cache, int64_t c_blk_stride, int64_t c_tok_stride,
                     int64_t c_head_stride, void* cache_scale, int64_t s_blk_stride,
                     int64_t s_tok_stride, int64_t s_head_stride, coopt_stream_t stream);

/*
 * The same swap for num_caches caches of one shape, dtype and strides -- the K and V caches
 * of every layer, which engine/kv_tier_manager.py:93-101 / 113-119 quantize / restore one
 * tensor at a time -- in one launch per 64 caches.  caches / cache_scales are host arrays of
 * device pointers (cache_scales NULL for bf16 caches); cache i swaps with the rows at
 * q + i * (num_ids * block_size * Hkv * D' * code bytes) and scale + i * num_ids * block_size
 * * Hkv, i.e. q / scale are contiguous [num_caches, num_ids, block_size, Hkv, D'] and
 * [num_caches, num_ids, block_size, Hkv].  Results are those of num_caches single calls.
 */
int coopt_kv_swap_out_caches(int bits, int cache_dtype, int num_caches, const void* const* caches,
                             const void* const* cache_scales, int64_t c_blk_stride,
                             int64_t c_tok_stride, int64_t c_head_stride, int64_t s_blk_stride,
                             int64_t s_tok_stride, int64_t s_head_stride,
                             const int64_t* block_ids, int num_ids, int block_size, int Hkv,
                             int D, int64_t num_blocks, void* q, void* scale,
                             coopt_stream_t stream);
int coopt_kv_swap_in_caches(int bits, int cache_dtype, int num_caches, const void* q,
                            const void* scale, const int64_t* block_ids, int num_ids,
                            int block_size, int Hkv, int D, int64_t num_blocks,
                            void* const* caches, void* const* cache_scales, int64_t c_blk_stride,
                            int64_t c_tok_stride, int64_t c_head_stride, int64_t s_blk_stride,
                            int64_t s_tok_stride, int64_t s_head_stride, coopt_stream_t stream);

/*
 * Block migration copy: for every pair i, block dst_ids[i] <- block src_ids[i] in every
 * region, in one launch per 32 regions.  Replaces the per-block copy_fn(src, dst) =
 * buf[dst].copy_(buf[src]) that BlockManager.migrate_out_of calls (engine/elastic.py:131,
 * engine/block_manager.py:165-187).
 *   regions   host array [num_regions][3] of int64 {device base address, bytes between
 *             consecutive block ids, bytes per block}: block b of a region is the byte range
 *             [base + b * stride, base + b * stride + bytes).  One region may be the whole
 *             block-major buffer [NB, L, 2, bs, Hkv, D] (engine/elastic.py:74-77), or one
 *             per-layer K/V cache or INT8 scale cache whose blocks are dense.  Base, stride
 *             and bytes must be multiples of 16, and 0 < bytes <= stride.
 *   src_ids, dst_ids  [num_pairs] int64 device arrays.  A pair with either id outside
 *             [0, num_blocks) is skipped.  Pairs are copied in no particular order, so no dst
 *             may be the src of another pair, and no two pairs may share a dst (a migration
 *             out of a set of blocks into free blocks outside it satisfies both).
 */
int coopt_kv_copy_blocks(const int64_t* regions, int num_regions, const int64_t* src_ids,
                         const int64_t* dst_ids, int num_pairs, int64_t num_blocks,
                         coopt_stream_t stream);

/*
 * Paged GQA verification attention.  Replaces flash_attn_varlen_func(q, k_cache, v_cache,
 * cu_seqlens_q, max_seqlen_q, seqused_k=seq_lens, max_seqlen_k, softmax_scale, causal=True,
 * block_table) at engine/model.py:244-247.  For sequence b with n = cu[b+1]-cu[b] query rows
 * and L = seq_lens[b] keys, query j and head h attend to keys [0, L - n + j] of KV head
 * h / (Hq/Hkv) (causal mask aligned bottom-right, engine/model.py:8-10).
 *
 *   q      [T, Hq, D] bf16 (q_tok_stride, q_head_stride, 1);  out likewise (o_tok_stride, ...)
 *   kv_dtype COOPT_DT_BF16: caches bf16 [NB, block_size, Hkv, D], k_scale/v_scale unused
 *            COOPT_DT_I8:   caches int8 codes, k_scale/v_scale fp16 [NB, block_size, Hkv].
 *                           K: every code is dequantised in the kernel to
 *                           bf16(float(code) * float(scale)), the value dequantize() gives,
 *                           so the scores use the reference's operands.  V: the codes enter
 *                           the PV product as exact fp16 integers and each key's V scale is
 *                           folded into its probability, rounded once to fp16 as
 *                           p * s_v * 2^-e (e a per-wave power of two that keeps the product
 *                           in fp16's normal range for every fp16 scale).  The output is
 *                           therefore not bit-equal to the bf16 path on the dequantised
 *                           cache; it stays within the INT8 tolerance of attention over it.
 *   block_table [B, bt_stride] int32; entries past ceil(L/block_size) are never read.
 *   Supported: D in {64, 128}; Hq/Hkv <= 64; block_size a power of two >= 16; B <= 65535.
 *   Query rows: up to 64 rows per (sequence, KV head), i.e. (Hq/Hkv) * max_seqlen_q <= 64
 *   (speculative verify and decode), run on the tuned path (contexts split over blocks).
 *   Longer items -- the prefill chunks the engine mixes into one batch with its verify items
 *   (engine/engine.py:414-420), or a long draft catch-up -- run in query windows of
 *   64/(Hq/Hkv) rows, each window one block over the keys its last row sees: correct at any
 *   length, not tuned for throughput (B * windows * Hkv < 2^24 blocks).  Callers must keep seq_lens <= max_seqlen_k, q rows per sequence
 *   <= max_seqlen_q and block ids in [0, num_blocks); the kernel clamps all three so a
 *   malformed call yields wrong rows but never an access outside its buffers.
 *   workspace: coopt_verify_attention_workspace() bytes (see above).
 *   Scheduling: when a batch of B <= 64 sequences has more (sequence, KV head) items than the
 *   GPU runs at once, the blocks take them longest first (whatever order the batch lists
 *   them in), so the long sequences start early instead of being left for last.
 */
size_t coopt_verify_attention_workspace(int B, int Hq, int Hkv, int D, int max_seqlen_q,
                                        int max_seqlen_k);
int coopt_verify_attention(int kv_dtype,
                           const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                           const void* k_cache, const void* v_cache,
                           int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                           const void* k_scale, const void* v_scale,
                           int64_t s_blk_stride, int64_t s_tok_stride, int64_t s_head_stride,
                           const int32_t* block_table, int64_t bt_stride,
                           const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                           int B, int Hq, int Hkv, int D, int block_size, int64_t num_blocks,
                           int max_seqlen_q, int max_seqlen_k, float softmax_scale,
                           void* out, int64_t o_tok_stride, int64_t o_head_stride,
                           void* workspace, size_t workspace_bytes, coopt_stream_t stream);

/*
 * The qkv epilogue and the verification attention of one layer in one launch: replaces
 * F.linear(h, qkv).split -> rotary_embedding(q, k) -> reshape_and_cache_flash(k, v) ->
 * flash_attn_varlen_func(q, ...) at engine/model.py:238-247 (what coopt_qkv_epilogue followed
 * by coopt_verify_attention do), bit for bit the same outputs and cache contents.  The block
 * of (sequence b, KV head h) reduces and rotates its rows' q heads straight into on-chip
 * memory, writes its rows' K and V of head h to the cache (INT8 quantised with cache_dtype
 * COOPT_DT_I8), then attends.
 *   qkv / part, ks, slice_stride, positions, cos, sin, table_stride, max_pos, slot_mapping:
 *       as coopt_qkv_epilogue (exactly one of qkv / part; part with 1 <= ks <= 4 slices);
 *       rows are the T = cu_seqlens_q[B] query rows.
 *   caches, scales, block_table, cu_seqlens_q, seq_lens, sizes, out, workspace: as
 *       coopt_verify_attention (kv_dtype the cache type); the caches are written here.
 * Contract: row j of sequence b writes key position seq_lens[b] - n_b + j of b's pages (its
 * slot_mapping entry points there, or is -1 for a padding row), as the reference writes a
 * step's tokens before attending over them; blocks read their new keys back only after
 * writing them.
 * Supported where coopt_verify_attention_qkv_supported() returns 1: one context split per
 * (sequence, KV head) at this B and max_seqlen_k, and (Hq/Hkv) * max_seqlen_q <= 32 (<= 16
 * with bf16 KV at head_dim 128).  Elsewhere the call returns COOPT_EINVAL; use the two calls.
 */
int coopt_verify_attention_qkv_supported(int kv_dtype, int B, int Hq, int Hkv, int D,
                                         int max_seqlen_q, int max_seqlen_k);
int coopt_verify_attention_qkv(int kv_dtype, const void* qkv, int64_t qkv_tok_stride,
                               const float* part, int ks, int64_t slice_stride,
                               const int64_t* positions, const void* cos, const void* sin,
                               int64_t table_stride, int max_pos, const int64_t* slot_mapping,
                               void* k_cache, void* v_cache,
                               int64_t c_blk_stride, int64_t c_tok_stride, int64_t c_head_stride,
                               void* k_scale, void* v_scale,
                               int64_t s_blk_stride, int64_t s_tok_stride, int64_t s_head_stride,
                               const int32_t* block_table, int64_t bt_stride,
                               const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                               int B, int Hq, int Hkv, int D, int block_size, int64_t num_blocks,
                               int max_seqlen_q, int max_seqlen_k, float softmax_scale,
                               void* out, int64_t o_tok_stride, int64_t o_head_stride,
                               void* workspace, size_t workspace_bytes, coopt_stream_t stream);

/*
 * Fused speculative acceptance for a batch (engine/spec_decode.py:20-49, looped over the
 * batch at engine/engine.py:437-446), with the random draws made explicit:
 *   temperature > 0:  p_i = softmax(target_i * (1/T)), q_i = softmax(draft_i * (1/T))
 *     (draft_kind 1: draft rows already hold q_i, fp32).  Draft i is accepted while
 *     u_accept[b,i] < min(1, p_i[d_i] / max(q_i[d_i], 1e-20)); k = first rejection (or g_b).
 *     The emitted token is drawn by inverse CDF with u_resample[b] from max(0, p_k - q_k)
 *     (normalised; p_k if it sums to 0) or, when all g_b drafts are accepted, from p_{g_b}:
 *     the smallest index j with cumsum(w)[j] > u * sum(w).
 *   temperature <= 0: greedy; argmax (first index on ties) per row, accept while equal.
 * Rows: sequence b's target rows are target_row0[b] + i (i <= g_b) of a row-major
 * [*, V] array with row stride target_row_stride (target_row0 NULL: b*(gamma_max+1));
 * its draft rows are draft_row0[b] + i (i < g_b) (NULL: b*gamma_max).
 * g_b = gamma_per_seq[b] (NULL: gamma_max), 0 <= g_b <= gamma_max.
 * Outputs: accepted_len[b] = k; out_tokens[b, 0..k] = d_0..d_{k-1}, token; the rest -1.
 * margin[b] (optional) = the smallest distance between a uniform and the boundary that
 * decided it (|u_i - ratio_i| for i <= k, and the inverse-CDF distance in probability
 * mass), so callers can report decisions within rounding of a boundary as ties.
 * logits_dtype COOPT_DT_F32 or COOPT_DT_BF16 (target and draft logits alike).
 */
size_t coopt_accept_sample_workspace(int B, int gamma_max, int V);
int coopt_accept_sample(int logits_dtype,
                        const void* target, int64_t target_row_stride, const int32_t* target_row0,
                        int draft_kind, const void* draft, int64_t draft_row_stride,
                        const int32_t* draft_row0,
                        const int32_t* draft_tokens, const int32_t* gamma_per_seq,
                        const float* u_accept, const float* u_resample, float temperature,
                        int B, int gamma_max, int V,
                        int32_t* accepted_len, int32_t* out_tokens, float* margin,
                        void* workspace, size_t workspace_bytes, coopt_stream_t stream);

/*
 * coopt_accept_sample without a workspace argument: no counterpart in the reference.  For
 * callers that cannot allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  Same arguments, kernels and results as
 * coopt_accept_sample; its workspace is a file-scope device array of
 * coopt_accept_sample_noalloc_max_bytes() bytes (2 MiB: B <= 512 at gamma_max 8 and V 128256,
 * or B <= 256 at V 262144), which each GPU holds until the process ends.  Sizes whose
 * coopt_accept_sample_workspace() exceeds it return COOPT_EWORKSPACE with a message.  It
 * allocates nothing and needs no clearing (the kernels initialise what they read); every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU (different streams or
 * host threads without ordering) race.
 */
size_t coopt_accept_sample_noalloc_max_bytes(void);
int coopt_accept_sample_noalloc(int logits_dtype,
                                const void* target, int64_t target_row_stride,
                                const int32_t* target_row0, int draft_kind, const void* draft,
                                int64_t draft_row_stride, const int32_t* draft_row0,
                                const int32_t* draft_tokens, const int32_t* gamma_per_seq,
                                const float* u_accept, const float* u_resample, float temperature,
                                int B, int gamma_max, int V,
                                int32_t* accepted_len, int32_t* out_tokens, float* margin,
                                coopt_stream_t stream);

/*
 * probs[r, :] = softmax(logits[r, :] * (1/T)) in fp32 (engine/spec_decode.py:16), for the
 * probabilities sample() returns.  logits F32 or BF16 with row stride in_stride.
 */
int coopt_softmax(int logits_dtype, const void* logits, int64_t in_stride, int64_t rows, int V,
                  float temperature, float* probs, int64_t out_stride, coopt_stream_t stream);

/*
 * The same probabilities for the rows a sampling call just drew from (engine/spec_decode.py:
 * 16, the probs sample() returns next to its tokens): it reads the row statistics that a
 * preceding coopt_accept_sample with gamma_max = 0 on the same logits, B, V, temperature and
 * workspace left there, stream-ordered before this call, so each element is read once and the
 * rows are spread over the whole GPU.  workspace_bytes >= coopt_accept_sample_workspace(B, 0, V).
 */
int coopt_sample_probs(int logits_dtype, const void* logits, int64_t in_stride, int B, int V,
                       float temperature, const void* workspace, size_t workspace_bytes,
                       float* probs, int64_t out_stride, coopt_stream_t stream);

/*
 * sample(logits, T) at T > 0 (engine/spec_decode.py:12-17) in two launches: tokens[r] is the
 * inverse-CDF draw of uniforms[r] from softmax(logits[r] * (1/T)), the same rule and margin as
 * coopt_accept_sample with gamma_max = 0 (which runs these launches too), and with probs
 * non-NULL the probabilities are written by the same second launch (one read of the logits
 * per launch, one write of the probabilities).  margin may be NULL.
 * workspace_bytes >= coopt_accept_sample_workspace(N, 0, V).
 */
int coopt_sample(int logits_dtype, const void* logits, int64_t row_stride, int N, int V,
                 float temperature, const float* uniforms, int32_t* tokens, float* margin,
                 float* probs, int64_t probs_stride, void* workspace, size_t workspace_bytes,
                 coopt_stream_t stream);

/*
 * Elementwise stages of the Llama forward around the verify path (the model the step
 * benchmark runs), fused as the reference's forward fuses them (engine/model.py:234-254).
 *
 * coopt_rms_norm: x, residual, weight, out bf16 [rows, hidden] (weight [hidden]).  With a
 *   residual (vLLM fused_add_rms_norm): residual := bf16(x + residual), then the norm reads it;
 *   without (vLLM rms_norm) it reads x.  out = bf16(w * bf16(r * rsqrt(mean(r^2) + eps))), the
 *   rounding points of the reference's rms_norm (engine/model.py:85-89).  out may alias x.
 * coopt_rope: in place on q [T, Hq, D] and k [T, Hkv, D] (strides as given, D contiguous),
 *   neox half-split rotation with bf16 cos/sin tables [max_pos, table_stride] indexed by
 *   positions[t] (engine/model.py:92-94, 120-127); positions are clamped to [0, max_pos).
 * coopt_silu_mul: out[t, j] = silu(gate_up[t, j]) * gate_up[t, F + j], bf16, F % 8 == 0.
 */
int coopt_rms_norm(const void* x, void* residual, const void* weight, void* out, int64_t rows,
                   int hidden, float eps, coopt_stream_t stream);
int coopt_rope(void* q, int64_t q_tok_stride, int64_t q_head_stride, void* k,
               int64_t k_tok_stride, int64_t k_head_stride, const int64_t* positions,
               const void* cos, const void* sin, int64_t table_stride, int max_pos, int T, int Hq,
               int Hkv, int D, coopt_stream_t stream);
int coopt_silu_mul(const void* gate_up, void* out, int64_t T, int F, coopt_stream_t stream);
/*
 * coopt_rms_norm with x given as the fp32 split-K partials of the linear layer that produced
 * it (coopt_linear_partials): x[row] = bf16(sum over k < ks, in order, of
 * part[k * slice_stride + row * hidden + :]) -- the value coopt_linear would have written --
 * then the fused add and the norm as coopt_rms_norm.  hidden <= 8192, 1 <= ks <= 16.
 */
/*
 * coopt_silu_mul with gate_up given as fp32 split-K partials (coopt_linear_partials of the
 * gate_up projection): gate_up[t] = bf16(sum over k < ks, in order, of
 * part[k * slice_stride + t * 2F + :]), then silu(gate) * up as coopt_silu_mul.  1 <= ks <= 16.
 */
int coopt_silu_mul_partials(const float* part, int ks, int64_t slice_stride, void* out,
                            int64_t T, int F, coopt_stream_t stream);
int coopt_rms_norm_partials(const float* part, int ks, int64_t slice_stride, void* residual,
                            const void* weight, void* out, int64_t rows, int hidden, float eps,
                            coopt_stream_t stream);

/*
 * Paged addressing of a batch of row runs on the device -- BlockManager.slot_mapping
 * (engine/block_manager.py:216-220: slot = table[p / bs] * bs + p % bs) and the positions and
 * seq_lens of build_batch (engine/batch.py:23-55), for the padded verify layout
 * (engine/cuda_graphs.py:76-104) where sequence b owns rows [b S, (b + 1) S).
 *   block_table [B, table_width] int32 (row stride table_stride); start [B] int64.
 *   positions [B S] = start[b] + j; slots [B S] int64; seq_lens [B] int32 = start[b] + S (NULL
 *   to skip).  slots = -1 for rows with j >= n_real[b] (n_real [B] int64, NULL = all real) and
 *   for block indices outside [0, table_width).
 */
int coopt_row_slots(const int32_t* block_table, int64_t table_stride, int table_width,
                    const int64_t* start, const int64_t* n_real, int B, int S, int block_size,
                    int64_t* positions, int64_t* slots, int32_t* seq_lens, coopt_stream_t stream);

/*
 * Linear layer at decode / verify row counts: y[M, N] = x[M, K] w[N, K]^T, bf16 in and out,
 * fp32 accumulation, no bias -- the projections of the reference's forward (F.linear at
 * engine/model.py:238, 248, 250, 253: qkv, o, gate_up, down; and the logits projection).
 *   x  [M, K] row stride ldx; w [N, K] row stride ldw (both 16-byte aligned, strides multiples
 *   of 8 elements); y [M, N] row stride ldy (8-byte aligned, a multiple of 4).
 *   1 <= M <= 256, K a multiple of 128, N a multiple of 4.
 *   workspace: coopt_linear_workspace(M, N, K) bytes (0 = none needed).  Large K is split over
 *   workgroups whose fp32 partial sums are added in a fixed order, so results are
 *   deterministic; the summation order differs from a library GEMM's (results agree to bf16
 *   rounding of the fp32 sum).
 */
size_t coopt_linear_workspace(int M, int N, int K);
/*
 * The split-K plan of coopt_linear for (M, N, K): *ks K slices, each a [*rows_padded, N] fp32
 * block of partial sums.  coopt_linear_partials runs the same kernel but leaves all ks slices
 * in the workspace (ks * rows_padded * N * 4 bytes, also when ks == 1) instead of reducing
 * them, for a consumer that reduces while it reads -- coopt_rms_norm_partials below.
 */
int coopt_linear_split(int M, int N, int K, int* ks, int* rows_padded);
int coopt_linear_partials(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N,
                          int K, void* workspace, size_t workspace_bytes, coopt_stream_t stream);
int coopt_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K,
                 void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                 coopt_stream_t stream);
/*
 * The same projections with the weight in tile-packed form, written once at model load by
 * coopt_linear_pack_weight (a layout for the MI355X memory system; the reference keeps F.linear's
 * row-major [N, K] weight, engine/model.py:238, 248, 253, which is the input here).
 *   coopt_linear_pack_weight: out (N * K bf16, 16-byte aligned) = w [N, K] (row stride ldw)
 *     as [N/16][K/128] tiles of 16 rows x 128 K; in tile (t, u), 16-byte chunk j * 64 + l holds
 *     w[16 t + l % 16][128 u + 32 j + 8 (l / 16), +8).  N a multiple of 16, K of 128.
 *   coopt_linear_packed / coopt_linear_partials_packed: coopt_linear / coopt_linear_partials
 *     with w_packed in place of (w, ldw); same plan, workspace and split, results bit-identical.
 */
int coopt_linear_pack_weight(const void* w, int64_t ldw, int N, int K, void* out,
                             coopt_stream_t stream);
int coopt_linear_packed(const void* x, int64_t ldx, const void* w_packed, int M, int N, int K,
                        void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                        coopt_stream_t stream);
int coopt_linear_partials_packed(const void* x, int64_t ldx, const void* w_packed, int M, int N,
                                 int K, void* workspace, size_t workspace_bytes,
                                 coopt_stream_t stream);
/*
 * The gate_up projection fused with SiLU-and-mul, engine/model.py:250-252
 * (silu_and_mul(F.linear(h, gate_up))), at draft and verify row counts:
 *   coopt_linear_pack_gate_up: out (2F * K bf16) = the [2F, K] gate_up weight packed as
 *     coopt_linear_pack_weight does, with gate and up tiles interleaved: packed tile 2s holds
 *     gate rows [16 s, +16), tile 2s + 1 up rows [F + 16 s, +16).  F a multiple of 16.
 *   coopt_linear_silu_supported(M, F, K): 1 when the fused path takes the shape (M <= 64 or
 *     129 <= M <= 160, 2F < 65536 and K not split by coopt_linear's plan), else 0.
 *   coopt_linear_silu_packed: y [M, F] (row stride ldy) = bf16(silu(g) * u) with
 *     g = bf16(x w_gate^T), u = bf16(x w_up^T) -- bit for bit what coopt_linear followed by
 *     coopt_silu_mul gives -- in one launch, no workspace.
 */
int coopt_linear_pack_gate_up(const void* w, int64_t ldw, int F, int K, void* out,
                              coopt_stream_t stream);
int coopt_linear_silu_supported(int M, int F, int K);
int coopt_linear_silu_packed(const void* x, int64_t ldx, const void* w_gu_packed, int M, int F,
                             int K, void* y, int64_t ldy, coopt_stream_t stream);

/*
 * Bookkeeping of one speculative step on the device, for the batch in slots [0, Bc) of a
 * decoder's state (engine/engine.py:338-470 for a batch in which every sequence decodes; the
 * reference walks Python lists on the host between launches).  One workgroup each; sizes up
 * to a few hundred sequences.  State per slot: live [Bc] uint8 (0/1), gamma [Bc] int64 (the
 * caller's draft length), n [Bc] int64 (tokens so far), dc [Bc] int64 (draft KV length,
 * draft_computed), hist [Bc][hist_stride] int64 (tokens; positions < max_len).
 *
 * coopt_spec_step_begin (engine/engine.py:354-389, 414-417): the step's uniforms u[0, nu) =
 * u_table row (*u_counter mod u_rows), then *u_counter += 1.  Per sequence, with lag = n - dc:
 * gamma_eff = gamma if live, gamma > 0 and lag <= 2 (speculate), else 0; the draft catch-up
 * (G > 0 only) starts at cu_start = dc (0 when not live) with cu_nreal = lag when speculating,
 * min(lag - 1, S_c) when lagging, 0 otherwise, tokens cu_tokens [Bc][S_c] = hist[start + j]
 * (clamped to max_len - 1), and cu_keep_rows [Bc] = b S_c + max(cu_nreal - 1, 0), the catch-up
 * row the first proposal is drawn from; proposal i = 1 .. G - 1 starts at pr_start[i - 1][b]
 * (row stride pr_stride) with pr_nreal = 1 while gamma_eff > i, draft_computed advancing by
 * that; the verify rows start at v_start = n - 1 with v_nreal = gamma_eff + 1 (0 and 0 when not
 * live) and token v_tokens[b][0] = hist[v_start] (v_tokens [Bc][S_t]); dc_final = draft_computed
 * after the draft phase.
 */
int coopt_spec_step_begin(const float* u_table, int64_t u_rows, int nu, int64_t* u_counter,
                          float* u, const uint8_t* live, const int64_t* gamma, const int64_t* n,
                          const int64_t* dc, const int64_t* hist, int64_t hist_stride,
                          int64_t max_len, int Bc, int G, int S_c, int S_t, int32_t* gamma_eff,
                          int64_t* cu_start, int64_t* cu_nreal, int64_t* cu_tokens,
                          int64_t* cu_keep_rows, int64_t* pr_start, int64_t* pr_nreal,
                          int64_t pr_stride, int64_t* v_start, int64_t* v_nreal,
                          int32_t* v_tokens, int64_t* dc_final, coopt_stream_t stream);

/*
 * After the proposals (engine/engine.py:414-417): proposals [S_t - 1][prop_stride] int32
 * (proposal i of sequence b at i * prop_stride + b) into v_tokens[b][1 + i] ([Bc][S_t]) and
 * the accept test's draft rows draft_tokens [Bc][S_t - 1].
 */
int coopt_spec_step_verify_tokens(const int32_t* proposals, int64_t prop_stride, int Bc, int S_t,
                                  int32_t* v_tokens, int32_t* draft_tokens, coopt_stream_t stream);

/*
 * After the accept (engine/engine.py:444-446, 455, 463-470): for each live sequence with
 * k = accepted_len (clamped to [0, S_t - 1]), hist[n + j] = tokens[b][j] for j <= k (positions
 * < max_len; tokens [Bc][S_t] int32), n += k + 1, dc = min(dc_final, n - 1) (the rollback:
 * num_computed = len - 1 and draft_computed clamped to it); *emitted += sum(k + 1),
 * *drafted += sum(gamma_eff), *accepted += sum(k) over the live sequences.
 */
int coopt_spec_step_commit(const uint8_t* live, const int32_t* accepted_len, const int32_t* tokens,
                           int S_t, const int32_t* gamma_eff, const int64_t* dc_final, int64_t* n,
                           int64_t* dc, int64_t* hist, int64_t hist_stride, int64_t max_len,
                           int64_t* emitted, int64_t* drafted, int64_t* accepted, int Bc,
                           coopt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* COOPT_AMD_H */
