/*
 * qwen3_model_ops.h — C ABI of the row-wise kernels around the attention
 * path in a Qwen3 decoder step (same library, libqwen3_attn.so, and the
 * same conventions and return codes as qwen3_attn.h).
 *
 * Reference interfaces replaced (file:line in uphome/Qwen3-engine-from-scratch)
 *   qwen3_add_rms_norm_bf16 <- RMSNorm.forward (qwen3/norm.py:22-26) together
 *                              with the residual add before it
 *                              (qwen3/decoder.py:49,55), the embedding lookup
 *                              feeding layer 0 (qwen3/model.py:65,212) and the
 *                              final norm (qwen3/model.py:184,217)
 *   qwen3_silu_mul_bf16     <- F.silu(gate) * up of Qwen3MLP.forward
 *                              (qwen3/mlp.py:31-36)
 *   qwen3_argmax_bf16       <- the greedy path of sample_tokens
 *                              (qwen3/sampling.py:256-258: logits.argmax(-1))
 *   qwen3_decode_linear_bf16 <- the nn.Linear projections of a decode step
 *                              (qkv_proj qwen3/attention.py:81, o_proj :187,
 *                              gate_up_proj / down_proj qwen3/mlp.py:34-36,
 *                              lm_head qwen3/model.py:241) for batches of at
 *                              most 64 rows, with the RMSNorm before them, the
 *                              residual add after them or the SwiGLU activation
 *                              between them folded in
 *   qwen3_decode_qkv_rope_bf16 <- input RMSNorm + qkv_proj + q_norm / k_norm +
 *                              apply_rotary_pos_emb of a decode step
 *                              (qwen3/decoder.py:47, attention.py:81-96) and the
 *                              decode K/V write (update_kv_batch_triton,
 *                              qwen3/kernels/paged_attention.py:353-377), one launch
 *   qwen3_embed_ss_bf16     <- the embedding lookup (qwen3/model.py:212) writing
 *                              the residual stream and its partial sums of squares
 *                              for the fused first norm
 *   qwen3_lm_head_argmax_bf16 <- the final norm, lm_head and greedy choice of a
 *                              decode step (qwen3/model.py:217,241 and
 *                              qwen3/sampling.py:256-258) in one pass over the
 *                              tied embedding, without the logits
 *   qwen3_page_in_bf16      <- the device writes of KVCachePool.alloc (zeroing a
 *                              reused block, qwen3/PagedKVcache.py:58-73) and of
 *                              PagedKVCache._allocate_block (the resident table
 *                              entry, :140-150), for a whole batch in one launch
 *   qwen3_sample_bf16       <- sample_tokens (qwen3/sampling.py:234-270) with the
 *                              fused top-p / Gumbel-max kernel of its fast path
 *                              (:112-178) and its torch fallback (:76-108):
 *                              temperature, top-k, top-p per row in one launch
 *   qwen3_sample_ws_bf16    <- the same sample_tokens, its row-streaming
 *                              passes spread over parallel workgroups
 *   qwen3_advance_seq_lens  <- the resident-length write of
 *                              PagedKVCache.advance_seq_len
 *                              (qwen3/PagedKVcache.py:216-219), one launch for
 *                              a whole decode batch
 */
#ifndef QWEN3_MODEL_OPS_H
#define QWEN3_MODEL_OPS_H

#include "qwen3_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Residual add + RMSNorm over rows of `hidden` bf16 values.
 * For output row i, source row r = row_index ? row_index[i] : i (int64):
 *   h          = x ? bf16(residual[r] + x[r]) : residual[r]
 *   out[i]     = bf16((fp32(h) * rsqrt(mean(h^2) + eps)) * weight)
 *   residual_out[i] = h              (skipped when residual_out is NULL)
 * residual_out may alias residual when row_index is NULL (in-place update of
 * the residual stream).  With x NULL and residual the embedding table,
 * row_index the token ids and src_rows the vocabulary size, this is the
 * embedding lookup fused with layer 0's input norm; a row_index entry outside
 * [0, src_rows) gives a zero row.  Row strides in elements; rows 16-byte
 * aligned; hidden a multiple of 8, at most 8192. */
int qwen3_add_rms_norm_bf16(const void* x, int64_t x_row_stride,
                            const void* residual, int64_t residual_row_stride,
                            void* residual_out, int64_t residual_out_row_stride,
                            const void* weight, float eps,
                            void* out, int64_t out_row_stride,
                            const int64_t* row_index, int64_t src_rows,
                            int64_t rows, int hidden, void* stream);

/* SwiGLU activation: gate_up (rows, 2*intermediate) holds gate then up;
 * out[r, j] = bf16(bf16(silu(gate[r, j])) * up[r, j]), silu(g) = g / (1 + e^-g).
 * intermediate a multiple of 8; rows 16-byte aligned. */
int qwen3_silu_mul_bf16(const void* gate_up, int64_t gate_up_row_stride,
                        void* out, int64_t out_row_stride,
                        int64_t rows, int intermediate, void* stream);

/* Greedy token choice: out[r] (int64) = index of the largest of the `vocab`
 * bf16 logits of row r; the first such index on ties; a NaN ranks above
 * every number (torch.argmax's rule). */
int qwen3_argmax_bf16(const void* logits, int64_t row_stride, int64_t rows,
                      int64_t vocab, int64_t* out, void* stream);

/* Decode-batch linear layer y = a @ W^T for M <= 64 rows; W (weight) is
 * nn.Linear's (out x in) row-major matrix, K its input width (a multiple of
 * 128), N the output columns (a multiple of 16).
 * Prologue: with ss_in NULL, a = x.  Otherwise x is the residual stream h and
 *   a = bf16((h * rsqrt(mean(h^2) + eps)) * norm_weight), with sum(h^2) of
 *   row r taken as the sum of ss_in[r * ss_in_tiles + t] over t (partial sums
 *   written by the kernel that produced h).
 * Epilogue (epilogue argument):
 *   0 store     y[r, n] = bf16(acc)
 *   1 residual  h' = bf16(residual[r, n] + bf16(acc)) into residual_out, and
 *               ss_out[r * (N / 16) + n / 16] = sum of h'^2 over those 16 columns
 *               (residual_out must not alias residual)
 *   2 silu      gate rows are weight rows [0, N), up rows [up_row, up_row + N):
 *               y[r, n] = bf16(bf16(silu(bf16(gate))) * bf16(up))
 * Results do not depend on timing (fixed summation order). */
int qwen3_decode_linear_bf16(const void* x, int64_t x_row_stride,
                             const float* ss_in, int ss_in_tiles,
                             const void* norm_weight, float eps,
                             const void* weight, int64_t weight_row_stride,
                             int M, int N, int K, int epilogue,
                             void* y, int64_t y_row_stride,
                             const void* residual, int64_t residual_row_stride,
                             void* residual_out, int64_t residual_out_row_stride,
                             float* ss_out, int up_row, void* stream);

/* Decode step of one layer up to attention, for M <= 64 tokens: with
 * a = RMSNorm(h) (rms from ss_in as in qwen3_decode_linear_bf16), qkv =
 * bf16(a @ qkv_weight^T) ((num_heads + 2 * num_kv_heads) * 128 rows: q heads,
 * k heads, v heads), then per token exactly the decode form of
 * qwen3_qk_norm_rope_decode_bf16: q and k heads RMS-normalised with their
 * weights (head_eps) and rotated at positions[t] (NULL: seq_lens[row]); q
 * stored to q_out (M, num_heads, 128), k and v written into the pool at
 * position seq_lens[row] of row row_ids[t] (NULL: t) through the block
 * table.  A position outside the tables gives a zero q row and no write.
 * K a multiple of 64, at most 4096; head_dim 128. */
int qwen3_decode_qkv_rope_bf16(const void* h, int64_t h_row_stride,
                               const float* ss_in, int ss_in_tiles,
                               const void* norm_weight, float eps,
                               const void* qkv_weight, int64_t weight_row_stride,
                               int M, int K, int num_heads, int num_kv_heads, int head_dim,
                               const void* q_norm_weight, const void* k_norm_weight,
                               float head_eps, const float* cos_table, const float* sin_table,
                               int64_t table_row_stride, int64_t table_rows,
                               const int64_t* positions,
                               void* q_out, const int64_t q_out_strides[2],
                               void* k_cache, const int64_t k_cache_strides[4],
                               void* v_cache, const int64_t v_cache_strides[4],
                               int64_t num_blocks, int layer_idx, int num_layers,
                               const int32_t* seq_lens, const int32_t* block_table,
                               int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
                               const int32_t* row_ids, int block_size, void* stream);

/* h_out[r] = embedding[ids[r]] (zero row for an id outside [0, vocab)) and
 * ss_out[r * (hidden / 16) + t] = sum of h^2 over columns 16t .. 16t + 15:
 * the input of the first decode_linear with a norm prologue. */
int qwen3_embed_ss_bf16(const int64_t* ids, const void* embedding,
                        int64_t embedding_row_stride, int64_t vocab, int hidden, int M,
                        void* h_out, int64_t h_row_stride, float* ss_out, void* stream);

/* Maps new pool blocks into the resident block table and zeroes them:
 * entries holds three int32 arrays of n: rows, then page columns, then block
 * ids.  block_table[rows[i] * bt_row_stride + cols[i]] = blocks[i] (skipped
 * when the row or column is out of range) and the block_elems bf16 values of
 * block blocks[i] in k_cache and in v_cache (the pool's contiguous per-block
 * chunk: layers x heads x slots x head_dim) are set to zero.  n <= 65535. */
int qwen3_page_in_bf16(int32_t* block_table, int64_t bt_row_stride, int64_t max_rows,
                       int64_t max_pages, const int32_t* entries, int n,
                       void* k_cache, void* v_cache, int64_t block_elems,
                       int64_t num_blocks, void* stream);

/* Samples one token per row of bf16 logits (out[r], int64), per-row
 * parameters as device arrays (NULL: temperature 0, top_k 0, top_p 1):
 *   temperature[r] <= 0  the first index of the largest logit (NaN highest);
 *   otherwise            among the top_k[r] largest logits (all when
 *                        top_k[r] <= 0 or > vocab), sorted descending with
 *                        ties by lower index, the leading positions whose
 *                        softmax(logit / temperature) mass before them is
 *                        <= top_p[r] (the first always), a token is drawn
 *                        with probability proportional to
 *                        exp(logit / temperature) (Gumbel-max over the kept
 *                        tokens; Philox4x32-10 keyed by seed and row).
 * NaN logits are never drawn.  One 1024-thread workgroup per row. */
int qwen3_sample_bf16(const void* logits, int64_t row_stride, int64_t rows, int64_t vocab,
                      const float* temperature, const int32_t* top_k, const float* top_p,
                      uint64_t seed, int64_t* out, void* stream);

/* qwen3_sample_bf16's draws, bit for bit, for batches too small to fill the
 * CUs with one workgroup per row (<= 128 rows): each row is split over 2-8
 * parts (8 for <= 32 rows, 4 for <= 64, 2 for <= 128, at most one per
 * 8,192 tokens); a workgroup per part finds the part's own top-k boundary
 * and keeps the tokens at or above it, and a second launch draws from the
 * union of those lists (it holds every token of the row's top k), falling
 * back to streaming the row when the lists overflow.  The launches meet in
 * a caller workspace of qwen3_sample_workspace_bytes(rows, vocab) bytes
 * (device, 16-byte aligned, no initialisation; calls that share one must
 * not overlap); 0 bytes means one part per row, and then, or with a NULL
 * workspace, this call is qwen3_sample_bf16.  A smaller workspace returns
 * QWEN3_EWORKSPACE with the size needed in the error message. */
size_t qwen3_sample_workspace_bytes(int64_t rows, int64_t vocab);
int qwen3_sample_ws_bf16(const void* logits, int64_t row_stride, int64_t rows, int64_t vocab,
                         const float* temperature, const int32_t* top_k, const float* top_p,
                         uint64_t seed, int64_t* out, void* workspace, size_t workspace_bytes,
                         void* stream);

/* seq_lens[row_ids[i]] += delta for i < n, except rows equal to skip_row
 * (a captured batch's padding row) and rows outside [0, max_rows).  Rows
 * other than skip_row must be distinct.  The host keeps its own copy of the
 * lengths; this keeps the resident table in step without a host write. */
int qwen3_advance_seq_lens(int32_t* seq_lens, int64_t max_rows, const int32_t* row_ids,
                           int n, int skip_row, int delta, void* stream);

/* Workspace (device, 16-byte aligned) that qwen3_lm_head_argmax_bf16 needs:
 * per-workgroup row maxima.  Its contents need no initialisation. */
size_t qwen3_lm_head_argmax_workspace_bytes(void);

/* Greedy decode head for M <= 64 rows: a = RMSNorm(h) with the rms taken
 * from ss_in (as qwen3_decode_linear_bf16's norm prologue) and norm_weight,
 * logits = bf16(a @ weight^T) over vocab rows of weight (M x vocab, never
 * stored), out[r] (int64) = the first index of the largest logit of row r
 * (NaN ranks highest, as qwen3_argmax_bf16).  K a multiple of 512, at most
 * 1024.  Two launches (one workgroup per CU, then the per-row reduction). */
int qwen3_lm_head_argmax_bf16(const void* h, int64_t h_row_stride, const float* ss_in,
                              int ss_in_tiles, const void* norm_weight, float eps,
                              const void* weight, int64_t weight_row_stride, int M, int vocab,
                              int K, void* workspace, size_t workspace_bytes, int64_t* out,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN3_MODEL_OPS_H */
