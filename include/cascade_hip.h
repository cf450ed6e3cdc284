/*
 * cascade_hip.h -- C ABI of libcascade_hip.so, the gfx950 (MI355X) kernels and
 * copy primitives behind the layer_streaming batch=1 decode path.
 *
 * Every entry point:
 *   - is extern "C", takes raw device / pinned-host pointers, int64 sizes and
 *     a HIP stream handle passed as void* (torch: Stream.cuda_stream);
 *   - returns 0 on success, a hipError_t value on a HIP failure, or one of the
 *     CASCADE_E* codes below for a rejected argument (nothing is launched
 *     then); cascade_error_string() names any of them;
 *   - never allocates or frees memory and never synchronises the host, except
 *     cascade_event_create / cascade_event_destroy / cascade_event_synchronize,
 *     whose whole purpose is that;
 *   - is called from one host thread per stream; kernels are enqueued on the
 *     stream given.
 *
 * bf16 buffers are uint16_t arrays; all weight matrices are row-major
 * [rows, K] with rows contiguous (the layout of the reference's packed
 * host arena and device slots, layer_streaming/plan.py:219-243,
 * layer_streaming/runtime.py:127-135).  Matrix, vector and cache pointers
 * must be 16-byte aligned and K a multiple of 8.
 *
 * Reference citations are file:line in lianghan224-cloud/Cascade-LLM.
 */
#ifndef CASCADE_HIP_H
#define CASCADE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: cascade_hbm_read takes a workgroup count; the one-launch decoder layer
   exports are gone.  3: cascade_decode_attention_fused_bf16 /
   _fused_at_bf16 added.  4: cascade_topk_f32 added.  5: the split-K
   workspace forms cascade_gemm_ws_bf16 / cascade_gemm_residual_ws_bf16 and
   cascade_gemm_workspace_bytes added. */
#define CASCADE_ABI_VERSION 5

/* Argument errors (no work enqueued). */
#define CASCADE_EINVAL 1001     /* null pointer, bad size or count */
#define CASCADE_EALIGN 1002     /* pointer or K not 16-byte / 8-element aligned */
#define CASCADE_ESHAPE 1003     /* shape outside what the kernels support */
#define CASCADE_EWORKSPACE 1004 /* workspace smaller than *_workspace_bytes() */
#define CASCADE_ESCRATCH 1005   /* shape beyond the library's static scratch */

int cascade_abi_version(void);
const char *cascade_error_string(int code);

/* ---------------------------------------------------------------- RMSNorm
 * y = w * bf16(x * rsqrt(mean(x^2) + eps)), fp32 statistics, bf16 output,
 * rows of length n (rows contiguous).
 * Replaces _rms_norm, layer_streaming/llama31.py:21-25 (used at :173-179,
 * :256-263, :325-329).                                                     */
int cascade_rmsnorm_bf16(const void *x, const void *weight, void *y,
                         int64_t rows, int64_t n, float eps, void *stream);

/* ------------------------------------------------------------------ GEMV
 * y[N] = bf16(W[N,K] . x[K]), fp32 accumulation.
 * Replaces F.linear with one token, layer_streaming/llama31.py:241-245.    */
int cascade_gemv_bf16(const void *w, const void *x, void *y, int64_t n,
                      int64_t k, void *stream);

/* y[N] = bf16(residual[N] + bf16(W . x)).  y may alias residual.
 * Replaces `residual + F.linear(...)` for o_proj and down_proj,
 * layer_streaming/llama31.py:246-251 and :272-279.                         */
int cascade_gemv_residual_bf16(const void *w, const void *x,
                               const void *residual, void *y, int64_t n,
                               int64_t k, void *stream);

/* Fused input RMSNorm + Q/K/V projections + RoPE + KV-cache write for one
 * token at one position.
 *   normalized = rmsnorm(x, norm_weight, eps)  (norm_weight NULL: x as is)
 *   q = rope(bf16(Wq . normalized))  -> q_out[nq]
 *   k = rope(bf16(Wk . normalized))  -> k_out[h * kv_head_stride + d]
 *   v =      bf16(Wv . normalized)   -> v_out[h * kv_head_stride + d]
 * Head dim is 128; nq, nk, nv are multiples of 128 and any of them may be 0
 * (matrix granularity sends q_proj, k_proj and v_proj as separate units).
 * rope_cos / rope_sin point at the 64 bf16 cos / sin values of this position
 * (the two halves of a head share them).  k_out / v_out point at position
 * `pos` of KV head 0 of this layer's cache.
 * Replaces F.linear q/k/v (layer_streaming/llama31.py:241-245), the rotary
 * embedding + apply_rotary_pos_emb (llama31.py:206-212; transformers
 * models/llama/modeling_llama.py:113-160) and SimpleKVCache.append
 * (llama31.py:44-50).                                                       */
int cascade_qkv_rope_bf16(const void *wq, const void *wk, const void *wv,
                          int64_t nq, int64_t nk, int64_t nv, int64_t k,
                          const void *x, const void *norm_weight, float eps,
                          const void *rope_cos, const void *rope_sin,
                          void *q_out, void *k_out, void *v_out,
                          int64_t kv_head_stride, void *stream);
/* The same for a decode step whose position is held on the device (so that
 * one captured HIP graph of the step serves every token): the position is
 * p = *length - 1, clamped to [0, capacity).  rope_cos_table /
 * rope_sin_table are the [capacity, 64] bf16 tables (row p is used);
 * k_cache / v_cache point at position 0 of KV head 0 of this layer's cache,
 * kv_head_stride >= capacity * 128; K / V land at position p.  length is an
 * 8-byte aligned device int64 (cascade_decode_step_begin_bf16 advances it).
 * Same computation and replaced code as cascade_qkv_rope_bf16, with the
 * position the reference derives on the host per token (position_ids from
 * the cache length, llama31.py:131-143).                                   */
int cascade_qkv_rope_at_bf16(const void *wq, const void *wk, const void *wv,
                             int64_t nq, int64_t nk, int64_t nv, int64_t k,
                             const void *x, const void *norm_weight, float eps,
                             const void *rope_cos_table,
                             const void *rope_sin_table, void *q_out,
                             void *k_cache, void *v_cache,
                             int64_t kv_head_stride, const int64_t *length,
                             int64_t capacity, void *stream);

/* Fused post-attention RMSNorm + gate/up projections + SwiGLU:
 *   y[i] = bf16(bf16(silu(bf16(Wg[i] . n))) * bf16(Wu[i] . n)), i < n_half
 * norm_weight NULL: x is used as the normalized input.
 * Replaces llama31.py:252-275 (F.silu(F.linear(gate)), F.linear(up),
 * gate * up) for matrix_group / layer units, where gate and up are both
 * present.                                                                  */
int cascade_gate_up_swiglu_bf16(const void *w_gate, const void *w_up,
                                int64_t n_half, int64_t k, const void *x,
                                const void *norm_weight, float eps, void *y,
                                void *stream);

/* Matrix granularity halves of the same computation (gate_proj and up_proj
 * arrive as separate units, llama31.py:252-271):
 *   gate_silu: y[i] = bf16(silu(bf16(Wg[i] . n)))
 *   up_mul:    y[i] = bf16(gate[i] * bf16(Wu[i] . n))                        */
int cascade_gate_silu_bf16(const void *w_gate, int64_t n, int64_t k,
                           const void *x, const void *norm_weight, float eps,
                           void *y, void *stream);
int cascade_up_mul_bf16(const void *w_up, int64_t n, int64_t k, const void *x,
                        const void *norm_weight, float eps, const void *gate,
                        void *y, void *stream);

/* --------------------------------------------------------- decode attention
 * GQA attention of one query token over positions [0, L) of one layer's
 * cache: out[h*D + d] = bf16(softmax(q_h . K_g^T * scale) . V_g), g = h / G,
 * G = n_q_heads / n_kv_heads, D = head_dim (must be 128, G must be 4).
 * k_cache / v_cache point at position 0 of KV head 0; KV head g starts at
 * g * kv_head_stride elements, position p of a head at p * D.
 * Split over L; the workspace (zero-filled once by the caller, left zeroed
 * by every call) holds per-split partial softmax state.
 * Replaces _repeat_kv + F.scaled_dot_product_attention at decode,
 * layer_streaming/llama31.py:213-234.                                      */
size_t cascade_decode_attention_workspace_bytes(int64_t max_len,
                                                int64_t n_q_heads,
                                                int64_t n_kv_heads,
                                                int64_t head_dim);
int cascade_decode_attention_bf16(const void *q, const void *k_cache,
                                  const void *v_cache, int64_t kv_head_stride,
                                  int64_t len, int64_t n_q_heads,
                                  int64_t n_kv_heads, int64_t head_dim,
                                  float scale, void *out, void *workspace,
                                  size_t workspace_bytes, void *stream);
/* The same over positions [0, L) with L = *length (device int64, clamped to
 * [1, capacity]).  The launch shape follows capacity, so one captured
 * launch serves every L <= capacity; the workgroups split [0, L) as the
 * host-length form does (the result is bit-identical to it), and splits
 * past L's plan contribute nothing.  kv_head_stride >= capacity *
 * head_dim; workspace as above
 * (cascade_decode_attention_workspace_bytes(capacity, ...)).               */
int cascade_decode_attention_at_bf16(const void *q, const void *k_cache,
                                     const void *v_cache,
                                     int64_t kv_head_stride,
                                     const int64_t *length, int64_t capacity,
                                     int64_t n_q_heads, int64_t n_kv_heads,
                                     int64_t head_dim, float scale, void *out,
                                     void *workspace, size_t workspace_bytes,
                                     void *stream);

/* The two forms above with the split merge inside the attention launch: one
 * launch instead of two, results bit-identical to theirs.  The splits of KV
 * head g all run on XCD g (a workgroup serves the head numbered by the XCC
 * id it runs on; workgroups are dealt round-robin over the XCDs), and the
 * last of them to finish merge the head's outputs through that XCD's L2.  Needs
 * n_kv_heads == 8 (one KV head per XCD of an MI355X) and at least 8 splits
 * (len > 224; the _at form: capacity > 224); other shapes return
 * CASCADE_ESHAPE.  sync: CASCADE_DECODE_ATTENTION_SYNC_BYTES of device
 * memory, zero-filled once by the caller and left zeroed by every call that
 * completes; calls sharing one sync buffer must not overlap.  error_flag: a
 * device int32 into which the launch ors CASCADE_ATTN_EPLACEMENT (the
 * device did not deal the workgroups evenly over 8 XCDs) or
 * CASCADE_ATTN_ETIMEOUT (a merge wait ran out); after either, the outputs
 * are invalid and sync must be zero-filled again.  Workspace as for the
 * forms above.
 * Replaces the same reference code (llama31.py:213-234).                   */
#define CASCADE_DECODE_ATTENTION_SYNC_BYTES 1024
#define CASCADE_ATTN_EPLACEMENT 2
#define CASCADE_ATTN_ETIMEOUT 4
int cascade_decode_attention_fused_bf16(const void *q, const void *k_cache,
                                        const void *v_cache,
                                        int64_t kv_head_stride, int64_t len,
                                        int64_t n_q_heads, int64_t n_kv_heads,
                                        int64_t head_dim, float scale,
                                        void *out, void *workspace,
                                        size_t workspace_bytes, void *sync,
                                        int32_t *error_flag, void *stream);
int cascade_decode_attention_fused_at_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, const int64_t *length, int64_t capacity,
    int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim, float scale,
    void *out, void *workspace, size_t workspace_bytes, void *sync,
    int32_t *error_flag, void *stream);

/* The same computation as cascade_decode_attention_bf16 with no workspace
 * argument and no allocation of any kind: the split partials live in a
 * static device array of the library (one copy per GPU, about 1 MiB, held
 * until the process ends), sized for n_kv_heads <=
 * CASCADE_DECODE_ATTENTION_NOALLOC_MAX_KV_HEADS; larger shapes return
 * CASCADE_ESCRATCH.  Results are bit-identical to
 * cascade_decode_attention_bf16 (same kernels, same split plan).  Every call
 * on one GPU shares that array: calls that overlap on one GPU (two streams,
 * or two host threads) race and must be serialised by the caller.  The first
 * call on a GPU looks the array's device address up (hipGetSymbolAddress);
 * later calls only read the cached address.
 * No counterpart in the reference: this is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).                                                  */
#define CASCADE_DECODE_ATTENTION_NOALLOC_MAX_KV_HEADS 8
int cascade_decode_attention_noalloc_bf16(const void *q, const void *k_cache,
                                          const void *v_cache,
                                          int64_t kv_head_stride, int64_t len,
                                          int64_t n_q_heads, int64_t n_kv_heads,
                                          int64_t head_dim, float scale,
                                          void *out, void *stream);

/* ------------------------------------------------------ prefill (M > 1)
 * MFMA GEMMs over the token rows of a prefill call: Y[M, N] =
 * epilogue(X[M, K] . W[N, K]^T), X row-major [M, K] (already normalised:
 * run cascade_rmsnorm_bf16 over the rows first), W row-major [N, K],
 * fp32 accumulation, K a multiple of 64, M >= 1, any N >= 1 (the fused
 * SwiGLU GEMM needs n_half a multiple of 64, the QKV GEMM whole heads).
 * The epilogues round at the same points as the GEMV family above.  Each
 * replaces F.linear with a [1, S, K] input, layer_streaming/llama31.py:
 * 241-279, when the call carries S > 1 tokens.                             */
int cascade_gemm_bf16(const void *x, const void *w, void *y, int64_t m,
                      int64_t n, int64_t k, void *stream);
/* y[M, N] = bf16(residual + bf16(X . W^T)); y may alias residual
 * (o_proj / down_proj, llama31.py:246-251, :272-279).                      */
int cascade_gemm_residual_bf16(const void *x, const void *w,
                               const void *residual, void *y, int64_t m,
                               int64_t n, int64_t k, void *stream);
/* The same two products with a workspace: where 256-row tiles would keep at
 * most half of the device's CUs busy (M > 16 rows, N a multiple of 8,
 * K a multiple of 64; 17..1024 prompt rows over N = 4096 with K = 14336,
 * down_proj, and 17..128 rows with K = 4096, o_proj), K is
 * split over up to 8 groups of workgroups writing fp32 partials into the
 * workspace, which a second launch sums in split order before the
 * epilogue (same rounding points; the sum's association may move a result
 * by one bf16 place against the one-pass form).  Elsewhere they run the
 * one-pass GEMM and the workspace is not touched.  The workspace needs
 * cascade_gemm_workspace_bytes(m, n, k) bytes for the current device (0:
 * no split for this shape; a null workspace is then accepted), 16-byte
 * aligned; calls sharing one workspace must be ordered on one stream.
 * Replace the same F.linear calls as the forms above.                     */
size_t cascade_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k);
int cascade_gemm_ws_bf16(const void *x, const void *w, void *y, int64_t m,
                         int64_t n, int64_t k, void *workspace,
                         size_t workspace_bytes, void *stream);
int cascade_gemm_residual_ws_bf16(const void *x, const void *w,
                                  const void *residual, void *y, int64_t m,
                                  int64_t n, int64_t k, void *workspace,
                                  size_t workspace_bytes, void *stream);
/* fp32 y[M, N] = X . W^T, not rounded: the resident LM head over every
 * position, F.linear(normalized, lm_head).float() (llama31.py:330-334).    */
int cascade_gemm_f32out_bf16(const void *x, const void *w, float *y,
                             int64_t m, int64_t n, int64_t k, void *stream);
/* y = bf16(bf16(silu(bf16(X . Wg^T))) * bf16(X . Wu^T)), y [M, n_half]
 * (llama31.py:252-275, gate and up in one unit).                           */
int cascade_gate_up_swiglu_gemm_bf16(const void *x, const void *w_gate,
                                     const void *w_up, void *y, int64_t m,
                                     int64_t n_half, int64_t k, void *stream);
/* Matrix-granularity halves: y = bf16(silu(bf16(X . Wg^T))) and
 * y = bf16(gate * bf16(X . Wu^T)).                                         */
int cascade_gate_silu_gemm_bf16(const void *x, const void *w_gate, void *y,
                                int64_t m, int64_t n, int64_t k, void *stream);
int cascade_up_mul_gemm_bf16(const void *x, const void *w_up,
                             const void *gate, void *y, int64_t m, int64_t n,
                             int64_t k, void *stream);
/* Q/K/V projections of M tokens + RoPE + KV-cache write.  Row r is the
 * token at position pos0 + r (RoPE) and cache slot slot0 + r.  q rows go to
 * q_out [M, nq]; K / V head h of row r to k_out / v_out + h *
 * kv_head_stride + (slot0 + r) * 128.  rope_cos / rope_sin are [positions,
 * 64] bf16 tables with rope_positions rows (pos0 + M <= rope_positions);
 * kv_head_stride >= (slot0 + M) * 128.  Any of nq, nk, nv may be 0.
 * Replaces F.linear q/k/v, the rotary embedding and SimpleKVCache.append of
 * the prefill call (llama31.py:44-50, :206-218, :241-245).                 */
int cascade_qkv_rope_gemm_bf16(const void *x, int64_t m, const void *wq,
                               const void *wk, const void *wv, int64_t nq,
                               int64_t nk, int64_t nv, int64_t k,
                               const void *rope_cos, const void *rope_sin,
                               int64_t rope_positions, int64_t pos0,
                               void *q_out, void *k_out, void *v_out,
                               int64_t kv_head_stride, int64_t slot0,
                               void *stream);
/* Causal GQA attention of `tokens` query rows q [tokens, n_q_heads * 128]:
 * query row t (cache slot past + t) attends to positions [0, past + t] of
 * the layer cache (layout as cascade_decode_attention_bf16), out [tokens,
 * n_q_heads * 128] bf16.  head_dim 128, n_q_heads = 4 n_kv_heads,
 * past + tokens <= 2^24.
 * Replaces _repeat_kv + F.scaled_dot_product_attention(is_causal=True),
 * llama31.py:213-229 (the reference's prefill has past = 0).               */
int cascade_prefill_attention_bf16(const void *q, const void *k_cache,
                                   const void *v_cache, int64_t kv_head_stride,
                                   int64_t past, int64_t tokens,
                                   int64_t n_q_heads, int64_t n_kv_heads,
                                   int64_t head_dim, float scale, void *out,
                                   void *stream);

/* ------------------------------------------------------ LM head + top-k
 * One vocabulary chunk: logits[r] = W[r] . h (fp32, not rounded to bf16) for
 * rows r < rows, then an exact running top-k over everything seen since the
 * last call with first_chunk = 1.  Order: value descending, index ascending;
 * -0.0 == +0.0; NaN ranks highest.  After every call out_values[0..top_k) /
 * out_indices[0..top_k) hold the running result (global row index =
 * row_offset + r; entries beyond the rows seen so far are -inf / -1).
 * logits_out (nullable) receives the chunk's fp32 logits (logits_out[r]).
 * 1 <= top_k <= 64.  The workspace (zero-filled once by the caller) carries
 * the running list between calls on the same stream.
 * Replaces the per-chunk F.linear(...).float() + torch.topk + merge_topk of
 * VocabStreamingRuntime.lm_head_topk, layer_streaming/vocab.py:239-263 and
 * merge_topk vocab.py:11-32; with one chunk covering the whole vocabulary it
 * replaces the resident head, llama31.py:330-339.                          */
size_t cascade_lm_head_workspace_bytes(int64_t rows, int64_t top_k);
int cascade_lm_head_topk_bf16(const void *w, int64_t rows, int64_t k,
                              int64_t row_offset, const void *h, int64_t top_k,
                              int first_chunk, float *logits_out,
                              void *workspace, size_t workspace_bytes,
                              float *out_values, int64_t *out_indices,
                              void *stream);
/* The same exact top-k over a row of fp32 logits already in memory
 * (logits[0..rows), indices 0..rows-1; same order, ties and NaN rule),
 * with no running list: out_values / out_indices receive the row's top_k.
 * The workspace is one of cascade_lm_head_workspace_bytes(rows, top_k)
 * bytes (no zero-fill needed).  Replaces torch.topk(state.logits[:, -1:, :],
 * k) of the resident finish after its F.linear over every position,
 * layer_streaming/llama31.py:335-339.                                      */
int cascade_topk_f32(const float *logits, int64_t rows, int64_t top_k,
                     void *workspace, size_t workspace_bytes,
                     float *out_values, int64_t *out_indices, void *stream);

/* ----------------------------------------------------------- embedding
 * out[i, :] = table[ids[i], :] for i < n_ids (ids are int64 on the device).
 * An id outside [0, vocab) yields a zero row and sets *error_flag to 1
 * (error_flag is a device int32, nullable).
 * Replaces F.embedding on the resident table, llama31.py:144-148.           */
int cascade_embedding_gather_bf16(const void *table, int64_t vocab,
                                  int64_t hidden, const int64_t *ids,
                                  int64_t n_ids, void *out, int32_t *error_flag,
                                  void *stream);
/* First launch of a decode step with a device-held position: out[:] =
 * table[ids[0], :] as above, then, with L = *length on entry (the cached
 * length), history[L] = ids[0] and *length = L + 1.  L outside
 * [0, capacity) leaves *length and history unchanged and sets *error_flag.
 * ids, length and history (int64 [capacity]) are 8-byte aligned device
 * pointers; error_flag is nullable.  With ids pointing at the previous
 * step's top-1 output, a captured step feeds itself, and history collects
 * the greedy token sequence by position.  Replaces the per-token embedding
 * and the host's token / position bookkeeping of the decode loop,
 * tools/run_llama31.py:105-121 and llama31.py:128-150.                     */
int cascade_decode_step_begin_bf16(const void *table, int64_t vocab,
                                   int64_t hidden, const int64_t *ids,
                                   void *out, int64_t *length,
                                   int64_t *history, int64_t capacity,
                                   int32_t *error_flag, void *stream);

/* ------------------------------------------------------- copy pipeline
 * Thin wrappers so the two-slot pipeline runs on hipMemcpyAsync + hipEvent:
 * replaces slot.copy_(source, non_blocking=True) and the ready/free events
 * of DoubleBufferRuntime.run, layer_streaming/runtime.py:155-160,194-230,
 * and the LM-head chunk copies, layer_streaming/vocab.py:216-239.
 * Events are opaque handles (hipEvent_t) stored in a uint64.               */
int cascade_memcpy_h2d_async(void *dst, const void *src, size_t bytes,
                             void *stream);
int cascade_memcpy_d2d_async(void *dst, const void *src, size_t bytes,
                             void *stream);
int cascade_event_create(uint64_t *event, int enable_timing);
int cascade_event_destroy(uint64_t event);
int cascade_event_record(uint64_t event, void *stream);
int cascade_stream_wait_event(void *stream, uint64_t event);
int cascade_event_synchronize(uint64_t event);
/* 0 = complete, 1 = not yet complete, else an error code. */
int cascade_event_query(uint64_t event);
int cascade_event_elapsed_ms(uint64_t start, uint64_t end, float *ms);

/* Host memcpy of `bytes` from src to dst (non-overlapping host memory)
 * with `threads` threads (1..64: the caller plus threads started for this
 * call and joined before it returns), 2 MiB pieces, non-temporal stores;
 * returns when the copy is complete.  No HIP call is made and nothing
 * outlives the call.
 * Replaces the pageable -> pinned staging copy of PinnedStagingWeightStore
 * (layer_streaming/weight_store.py:258-268) and of the streamed LM head
 * (layer_streaming/vocab.py:143-147).                                      */
int cascade_host_copy(void *dst, const void *src, size_t bytes, int threads);

/* The same copy through a caller-owned pool of threads - 1 helper threads,
 * for a caller that stages many units (the reference's staging store makes
 * one copy per transfer unit, weight_store.py:258-268).  numa_node >= 0
 * binds the helpers to that node's CPUs (those this process may use; none
 * left -> unbound); -1 leaves them unbound; a node that does not exist is
 * CASCADE_EINVAL.  Copies on one pool from several threads run one after
 * another.  Destroy joins the helpers; no copy may be running on it.
 * cascade_copy_pool_info reports the thread count (helpers + caller) and
 * how many CPUs the helpers are bound to (0 = unbound).                    */
int cascade_copy_pool_create(int threads, int numa_node, uint64_t *pool);
int cascade_copy_pool_copy(uint64_t pool, void *dst, const void *src,
                           size_t bytes);
int cascade_copy_pool_info(uint64_t pool, int *threads, int *bound_cpus);
int cascade_copy_pool_destroy(uint64_t pool);

/* ----------------------------------------------------------- measurement
 * Streaming-read kernel: reads `bytes` of device memory (nontemporal 16-byte
 * loads, eight in flight per thread, 32 KiB contiguous per workgroup and
 * step) and folds them into *sink; `blocks`
 * workgroups of 256 threads (0: the library's default of up to 4096).  Used
 * to measure achievable HBM read bandwidth (no reference counterpart; the
 * reference measures only H2D, h2d_driver_bench.c).
 * Plain device copy of `bytes`: the calibration kernel for HBM traffic
 * counters.                                                                */
int cascade_hbm_read(const void *src, size_t bytes, float *sink,
                     int64_t blocks, void *stream);
int cascade_device_copy(void *dst, const void *src, size_t bytes, void *stream);

/* Binds two timing events (either may be 0) to the calling thread's next
 * kernel launch through this library: the start event takes that kernel's
 * start time and the stop event its end time (hipExtLaunchKernel), so their
 * elapsed time is the kernel's own duration.  The launch consumes them; an
 * entry point that fails before launching leaves them pending, and
 * (0, 0) clears them.  For an entry point that launches several kernels
 * only the first is timed.  No reference counterpart: the reference brackets
 * calls with torch.cuda.Event pairs (benchmarks/llama31_8b_m1_bench.py:84-95),
 * which also time the dispatch.                                             */
int cascade_time_next_launch(uint64_t start_event, uint64_t stop_event);

#ifdef __cplusplus
}
#endif

#endif /* CASCADE_HIP_H */
