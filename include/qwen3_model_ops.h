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

/* seq_lens[row_ids[i]] += delta for i < n, except rows equal to skip_row
 * (a captured batch's padding row) and rows outside [0, max_rows).  Rows
 * other than skip_row must be distinct.  The host keeps its own copy of the
 * lengths; this keeps the resident table in step without a host write. */
int qwen3_advance_seq_lens(int32_t* seq_lens, int64_t max_rows, const int32_t* row_ids,
                           int n, int skip_row, int delta, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN3_MODEL_OPS_H */
