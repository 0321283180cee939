/*
 * qwen3_attn.h — C ABI of the MI355X (gfx950) attention hot path of the
 * Qwen3 inference engine: paged decode attention, varlen causal prefill
 * attention, and the paged KV-cache slot writes.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers (HBM) unless stated otherwise; the
 *     library never allocates, frees or synchronises.  Work is enqueued on
 *     `stream` (a hipStream_t passed as void*; NULL = the null stream), so a
 *     caller inside stream capture records the launches into its graph.
 *   - Tensors are bf16 (raw 16-bit storage).  Strides are in ELEMENTS, not
 *     bytes; the innermost (head_dim) stride is always 1.
 *   - Indices into the resident tables are int32, as the reference keeps them.
 *   - Every entry point returns 0 on success, a negative QWEN3_E* code when an
 *     argument is rejected before anything is launched, or the positive
 *     hipError_t of a failed launch.  qwen3_attn_last_error() returns a
 *     human-readable message for the calling thread's last failure.
 *   - Out-of-range page ids, row ids and slots read from device tables are
 *     skipped by the kernels (never dereferenced), so a corrupt table cannot
 *     make a kernel read or write outside the buffers it was given.
 *   - Entry points that write into the pool take its layer count
 *     (num_layers) and reject layer_idx outside [0, num_layers) before
 *     launching anything.
 *
 * Reference interfaces replaced (file:line in uphome/Qwen3-engine-from-scratch)
 *   qwen3_paged_decode_bf16    <- paged_attention_decode_triton
 *                                 (qwen3/kernels/paged_attention.py:132-178)
 *                                 + paged_attn_decode_kernel (:27-129)
 *   qwen3_kv_write_decode_bf16 <- update_kv_batch_triton
 *                                 (qwen3/kernels/paged_attention.py:353-377)
 *                                 + update_kv_batch_kernel (:292-350)
 *   qwen3_kv_write_range_bf16  <- PagedKVCache.update advanced-indexing write
 *                                 (qwen3/PagedKVcache.py:177-214)
 *   qwen3_kv_write_slots_bf16  <- the per-request B-loop of PagedKVCache.update
 *                                 in batched prefill (qwen3/attention.py:160-161)
 *                                 collapsed into one slot-mapped launch
 *   qwen3_varlen_prefill_bf16  <- flash_attention_prefill
 *                                 (qwen3/kernels/flash_attention_varlen.py:126-194)
 *                                 + flash_attention_varlen_kernel (:25-123)
 *   qwen3_qk_norm_rope_decode_bf16 / _slots_bf16
 *                              <- q_norm, k_norm, apply_rotary_pos_emb and the
 *                                 pool write that follows them
 *                                 (qwen3/attention.py:91-96, qwen3/norm.py:22-26,
 *                                 qwen3/rope.py:88-110 + the decode / prefill
 *                                 writes above), fused into one launch
 */
#ifndef QWEN3_ATTN_H
#define QWEN3_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWEN3_OK 0
#define QWEN3_EINVAL (-1)       /* bad shape / size / stride / null pointer */
#define QWEN3_EALIGN (-2)       /* pointer or stride breaks required alignment */
#define QWEN3_EUNSUPPORTED (-3) /* head_dim / block_size / group size not built */
#define QWEN3_EWORKSPACE (-4)   /* workspace missing or too small */

/* Message for the calling thread's last failed call ("" if none). */
const char* qwen3_attn_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int qwen3_attn_abi_version(void);

/* ------------------------------------------------------------------------
 * Paged decode attention (GQA), one query token per sequence.
 *
 * Replaces paged_attention_decode_triton
 * (qwen3/kernels/paged_attention.py:132-178): for each batch entry b,
 *   row = row_ids ? row_ids[b] : b
 *   L   = seq_lens[row] + seq_len_bias      (the reference passes bias = 1:
 *                                            seq_lens holds the pre-step
 *                                            length, :55)
 *   out[b, h, :] = softmax(scale * q[b, h, :] . K[0:L]^T) V[0:L]
 * where token t of the sequence lives in physical page
 * block_table[row * bt_row_stride + t / block_size] at slot t % block_size,
 * and query head h reads KV head h / (num_heads / num_kv_heads).
 *
 *   q          (B, num_heads, head_dim)     strides q_strides[0..1]
 *   k_cache    per-layer view (num_blocks, num_kv_heads, block_size, head_dim)
 *              strides k_strides[0..2] (the layer stride is folded into
 *              k_strides[0], as the reference's pool.k_buffer[:, layer] view)
 *   v_cache    same layout, strides v_strides[0..2]
 *   out        (B, num_heads, head_dim)     strides out_strides[0..1]
 *   block_table int32 (max_rows, max_pages), row stride bt_row_stride
 *   seq_lens   int32 (max_rows,)
 *   row_ids    int32 (B,) or NULL (identity)
 *   workspace  device scratch of at least qwen3_paged_decode_workspace_bytes()
 *              bytes, 16-byte aligned (split-KV partials); its size depends
 *              only on (B, num_heads, num_kv_heads, head_dim, max_pages,
 *              block_size) and the current device's CU count, never on the
 *              live lengths, so one launch shape serves a captured graph.
 *              Its contents need no initialisation.
 * Supported: head_dim 128, block_size a multiple of 16,
 *            num_heads / num_kv_heads in [1, 16]; q, K, V and out rows
 *            16-byte aligned (strides multiples of 8 elements).
 * Launches two kernels on `stream` (the attention pass and a small merge of
 * sequences split across waves).
 * ---------------------------------------------------------------------- */
size_t qwen3_paged_decode_workspace_bytes(int B, int num_heads, int num_kv_heads,
                                          int head_dim, int64_t max_pages, int block_size);

int qwen3_paged_decode_bf16(const void* q, const int64_t q_strides[2],
                            const void* k_cache, const int64_t k_strides[3],
                            const void* v_cache, const int64_t v_strides[3],
                            int64_t num_blocks,
                            const int32_t* block_table, int64_t bt_row_stride,
                            int64_t max_rows, int64_t max_pages,
                            const int32_t* seq_lens, int seq_len_bias,
                            const int32_t* row_ids,
                            void* out, const int64_t out_strides[2],
                            int B, int num_heads, int num_kv_heads, int head_dim,
                            int block_size, float scale,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/* Batch-invariant variant of qwen3_paged_decode_bf16: the same arguments and
 * attention, computed so that a sequence's output bits depend only on its
 * own q, K, V and length, never on the batch around it (the same alone, at
 * any batch size, at any row position; the engine's batched == serial
 * guarantee).  No counterpart in the reference, whose Triton kernel splits
 * by batch shape; its callers are serving loops that need reproducible
 * tokens whatever else is batched.
 *   Each sequence-head is cut into 256-token partitions from its first
 *   token; each partition's softmax state is computed on its own (16-token
 *   tiles in pairs, from its first tile), and the output is the left fold of
 *   the partition states in ascending order.  The batch only decides which
 *   wave owns which partitions; a sequence split across waves is handed on
 *   through the workspace with tickets (no wave waits for another).
 *   workspace  qwen3_paged_decode_invariant_workspace_bytes() bytes, 16-byte
 *              aligned: first the hand-off tickets (4 x 2048 x num_kv_heads
 *              bytes, rounded up to 256), which must be zero before the
 *              first call (every call leaves them zero; calls that share a
 *              workspace use one num_kv_heads and one stream), then one slot
 *              per 256-token partition of every (b, KV head) at the table's
 *              full row length (B x num_kv_heads x ceil(max_pages x
 *              block_size / 256) slots of G x (128 + 2) floats), plus
 *              4 x (B + 1) + 256 bytes.  Depends on the launch shape only.
 *   Launches the attention pass on `stream`, plus a merge kernel when a
 *   table row can hold more than 32 partitions (8,192 tokens) or B > 2048.
 * Costs more HBM time than qwen3_paged_decode_bf16 where sequences are
 * split across waves (partition states written and read back). */
size_t qwen3_paged_decode_invariant_workspace_bytes(int B, int num_heads, int num_kv_heads,
                                                    int head_dim, int64_t max_pages,
                                                    int block_size);
int qwen3_paged_decode_invariant_bf16(const void* q, const int64_t q_strides[2],
                                      const void* k_cache, const int64_t k_strides[3],
                                      const void* v_cache, const int64_t v_strides[3],
                                      int64_t num_blocks,
                                      const int32_t* block_table, int64_t bt_row_stride,
                                      int64_t max_rows, int64_t max_pages,
                                      const int32_t* seq_lens, int seq_len_bias,
                                      const int32_t* row_ids,
                                      void* out, const int64_t out_strides[2],
                                      int B, int num_heads, int num_kv_heads, int head_dim,
                                      int block_size, float scale,
                                      void* workspace, size_t workspace_bytes,
                                      void* stream);

/* Allocation-free variant of qwen3_paged_decode_bf16.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, results and kernels as qwen3_paged_decode_bf16
 * minus the workspace: the split-KV partials live in a static device array of
 * 24 MiB that each GPU running the library holds until the process ends
 * (resolved once per device on the first call there).  Serves batches up to
 * 2048 whose partials fit it: 2 x waves x (G x 516 + ...) bytes, about
 * 2.1 MB x G on a 256-CU MI355X, so G = num_heads / num_kv_heads <= 11 there;
 * larger shapes return QWEN3_EWORKSPACE with the size they would need.
 * Every call of this entry point on one GPU shares that GPU's array, which
 * keeps the last call's contents (nothing in it has to start at zero); calls
 * that overlap on one GPU (concurrent streams) race and must be serialised
 * by the caller.  The stream must belong to the current device.  Allocates
 * nothing (no hipMalloc, no hipFree). */
int qwen3_paged_decode_noalloc_bf16(const void* q, const int64_t q_strides[2],
                                    const void* k_cache, const int64_t k_strides[3],
                                    const void* v_cache, const int64_t v_strides[3],
                                    int64_t num_blocks,
                                    const int32_t* block_table, int64_t bt_row_stride,
                                    int64_t max_rows, int64_t max_pages,
                                    const int32_t* seq_lens, int seq_len_bias,
                                    const int32_t* row_ids,
                                    void* out, const int64_t out_strides[2],
                                    int B, int num_heads, int num_kv_heads, int head_dim,
                                    int block_size, float scale, void* stream);

/* ------------------------------------------------------------------------
 * Decode-form K/V slot write.
 *
 * Replaces update_kv_batch_triton (qwen3/kernels/paged_attention.py:353-377):
 * for each (b, h):
 *   row  = row_ids[b];  pos = seq_lens[row]
 *   phys = block_table[row * bt_row_stride + pos / block_size]
 *   k_cache[phys, layer_idx, h, pos % block_size, :] = k_new[b, h, :]
 *   v_cache[...same...]                              = v_new[b, h, :]
 *   k_new, v_new  (B, num_kv_heads, head_dim), strides *_new_strides[0..1]
 *                 (non-contiguous slices of a fused QKV output are fine)
 *   k_cache/v_cache  full pool (num_blocks, num_layers, num_kv_heads,
 *                 block_size, head_dim), strides *_cache_strides[0..3]
 * The copy is bit-exact.
 * ---------------------------------------------------------------------- */
int qwen3_kv_write_decode_bf16(const void* k_new, const int64_t k_new_strides[2],
                               const void* v_new, const int64_t v_new_strides[2],
                               void* k_cache, const int64_t k_cache_strides[4],
                               void* v_cache, const int64_t v_cache_strides[4],
                               int64_t num_blocks, int layer_idx, int num_layers,
                               const int32_t* seq_lens,
                               const int32_t* block_table, int64_t bt_row_stride,
                               int64_t max_rows, int64_t max_pages,
                               const int32_t* row_ids,
                               int B, int num_kv_heads, int head_dim,
                               int block_size, void* stream);

/* ------------------------------------------------------------------------
 * Range-form K/V slot write for one sequence (prefill of one request).
 *
 * Replaces the advanced-indexing write of PagedKVCache.update
 * (qwen3/PagedKVcache.py:197-214): for s in [0, num_tokens), h:
 *   pos  = start_pos + s
 *   phys = block_table_row[pos / block_size]
 *   k_cache[phys, layer_idx, h, pos % block_size, :] = k_new[s, h, :]
 *   k_new, v_new  (num_tokens, num_kv_heads, head_dim), strides
 *                 *_new_strides[0] (token) and [1] (head); the reference's
 *                 (1, Hkv, S, D) tensor passes its S stride as [0], its
 *                 head stride as [1]
 *   block_table_row  int32 (row_pages,) — one row of the resident table
 * ---------------------------------------------------------------------- */
int qwen3_kv_write_range_bf16(const void* k_new, const int64_t k_new_strides[2],
                              const void* v_new, const int64_t v_new_strides[2],
                              void* k_cache, const int64_t k_cache_strides[4],
                              void* v_cache, const int64_t v_cache_strides[4],
                              int64_t num_blocks, int layer_idx, int num_layers,
                              const int32_t* block_table_row, int64_t row_pages,
                              int64_t start_pos, int64_t num_tokens,
                              int num_kv_heads, int head_dim, int block_size,
                              void* stream);

/* ------------------------------------------------------------------------
 * Slot-mapped K/V write (batched prefill).
 *
 * For t in [0, num_tokens), h:  slot = slot_mapping[t];
 *   if slot < 0 the token is skipped (padding), otherwise
 *   k_cache[slot / block_size, layer_idx, h, slot % block_size, :] = k_new[t, h, :]
 * slot_mapping is int64 (num_tokens,).  Equivalent, per request, to the
 * write of PagedKVCache.update (qwen3/PagedKVcache.py:197-214) with
 * slot = phys * block_size + offset.
 * ---------------------------------------------------------------------- */
int qwen3_kv_write_slots_bf16(const void* k_new, const int64_t k_new_strides[2],
                              const void* v_new, const int64_t v_new_strides[2],
                              void* k_cache, const int64_t k_cache_strides[4],
                              void* v_cache, const int64_t v_cache_strides[4],
                              int64_t num_blocks, int layer_idx, int num_layers,
                              const int64_t* slot_mapping, int64_t num_tokens,
                              int num_kv_heads, int head_dim, int block_size,
                              void* stream);

/* ------------------------------------------------------------------------
 * Varlen flash-attention prefill (packed sequences, GQA, causal).
 *
 * Replaces flash_attention_prefill
 * (qwen3/kernels/flash_attention_varlen.py:126-194): sequence s occupies
 * packed rows [cu_seqlens[s], cu_seqlens[s+1]); query row i of a sequence
 * attends keys j <= i of the same sequence (all j when causal == 0);
 * query head h reads KV head h / (num_heads / num_kv_heads).
 *   q, o      (total_tokens, num_heads, head_dim),    strides *_strides[0..1]
 *   k, v      (total_tokens, num_kv_heads, head_dim), strides *_strides[0..1]
 *   cu_seqlens int32 (num_seqs + 1,) on the device
 *   max_seqlen host-side upper bound of the sequence lengths (sizes the grid;
 *             the reference syncs cu_seqlens to the host to get it, :177-178).
 *             Contract: no sequence is longer.  Rows of a longer sequence
 *             past the first max_seqlen rounded up to the kernel's query
 *             tile are not written; a larger bound only costs empty work
 *             items and gives the same bits.
 *   workspace  optional (NULL: every item runs whole in one workgroup):
 *             qwen3_varlen_prefill_workspace_bytes() bytes (69 MB on a
 *             256-CU device: the size follows the current device's CU
 *             count) of device memory, zeroed before its first use; every
 *             call leaves its counters and tickets at zero.  With it a batch
 *             large enough for eight-wave workgroups has its work items
 *             dealt from counters as workgroups finish (heaviest first), and
 *             a batch with fewer work items than resident workgroups is cut
 *             into equal ranges of key tiles, one per workgroup; an item
 *             whose tiles span several ranges leaves one partial softmax
 *             state per range in the workspace and the last part to arrive
 *             folds them in key order (no part waits for another; the same
 *             bits whichever part arrives last).  Items of at most four key
 *             tiles (prompts of at most 256 tokens) are never cut.
 *             Concurrent calls need separate workspaces.
 * Supported: head_dim 128, num_heads / num_kv_heads in [1, 16].
 * ---------------------------------------------------------------------- */
size_t qwen3_varlen_prefill_workspace_bytes(void);

int qwen3_varlen_prefill_bf16(const void* q, const int64_t q_strides[2],
                              const void* k, const int64_t k_strides[2],
                              const void* v, const int64_t v_strides[2],
                              void* o, const int64_t o_strides[2],
                              const int32_t* cu_seqlens, int num_seqs,
                              int max_seqlen, int64_t total_tokens,
                              int num_heads, int num_kv_heads, int head_dim,
                              float scale, int causal, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Fused pre-attention step: QK-RMSNorm + RoPE + K/V pool write.
 *
 * Replaces, in one launch, q_norm / k_norm (qwen3/attention.py:91-92 with
 * qwen3/norm.py:22-26), apply_rotary_pos_emb (qwen3/attention.py:95-96,
 * qwen3/rope.py:88-110) and the pool write that follows
 * (update_kv_batch_triton, qwen3/kernels/paged_attention.py:292-377, for
 * decode; PagedKVCache.update, qwen3/PagedKVcache.py:177-214, for prefill).
 * Per head row: n = bf16((fp32(x) * rsqrt(mean(x^2) + eps)) * w);
 * out = bf16(bf16(n * bf16(cos[pos])) + bf16(rotate_half(n) * bf16(sin[pos])))
 * with rotate_half pairing element i with i + head_dim / 2.  V is copied to
 * the pool unchanged.
 *   q, k, v     (tokens, heads, head_dim) bf16 views (e.g. slices of the
 *               fused QKV projection), strides *_strides[0..1]
 *   q_weight, k_weight  (head_dim,) bf16 RMSNorm weights
 *   cos_table, sin_table (table_rows, head_dim) fp32, row stride
 *               table_row_stride (the model's RoPE tables; positions outside
 *               [0, table_rows) give zero q/k rows and no pool write)
 *   q_out       (tokens, num_heads, head_dim) bf16
 *   k_cache, v_cache  pool (num_blocks, num_layers, num_kv_heads, block_size,
 *               head_dim) with strides *_strides[0..3]; layer layer_idx
 * Supported: head_dim 128; rows 16-byte aligned.
 * ---------------------------------------------------------------------- */

/* Decode form: token b is request row_ids[b] (NULL: b); it is written at
 * position seq_lens[row] (the length before this step) through the resident
 * block table, as in qwen3_kv_write_decode_bf16, and rotated at
 * positions[b] (int64), the position_ids the reference passes
 * (qwen3/model.py:76-78, qwen3/graph_runner.py:190, bench_batched.py:182); positions NULL:
 * rotated at seq_lens[row] too, which is what every reference driver
 * passes. */
int qwen3_qk_norm_rope_decode_bf16(const void* q, const int64_t q_strides[2],
                                   const void* k, const int64_t k_strides[2],
                                   const void* v, const int64_t v_strides[2],
                                   const void* q_weight, const void* k_weight, float eps,
                                   const float* cos_table, const float* sin_table,
                                   int64_t table_row_stride, int64_t table_rows,
                                   void* q_out, const int64_t q_out_strides[2],
                                   void* k_cache, const int64_t k_cache_strides[4],
                                   void* v_cache, const int64_t v_cache_strides[4],
                                   int64_t num_blocks, int layer_idx, int num_layers,
                                   const int32_t* seq_lens, const int32_t* block_table,
                                   int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
                                   const int32_t* row_ids, const int64_t* positions, int B,
                                   int num_heads, int num_kv_heads, int head_dim,
                                   int block_size, void* stream);

/* Slot form (prefill): token t has RoPE position positions[t] (int64) and
 * pool slot slot_mapping[t] = block * block_size + offset (int64; negative
 * or NULL: no pool write).  k_out (nullable) receives the normalised,
 * rotated K for the prefill attention kernel. */
int qwen3_qk_norm_rope_slots_bf16(const void* q, const int64_t q_strides[2],
                                  const void* k, const int64_t k_strides[2],
                                  const void* v, const int64_t v_strides[2],
                                  const void* q_weight, const void* k_weight, float eps,
                                  const float* cos_table, const float* sin_table,
                                  int64_t table_row_stride, int64_t table_rows,
                                  const int64_t* positions, const int64_t* slot_mapping,
                                  void* q_out, const int64_t q_out_strides[2],
                                  void* k_out, const int64_t k_out_strides[2],
                                  void* k_cache, const int64_t k_cache_strides[4],
                                  void* v_cache, const int64_t v_cache_strides[4],
                                  int64_t num_blocks, int layer_idx, int num_layers,
                                  int64_t num_tokens,
                                  int num_heads, int num_kv_heads, int head_dim,
                                  int block_size, void* stream);

/* ------------------------------------------------------------------------
 * Streaming read reference (no counterpart in the reference engine; for the
 * measurement of the HBM-bound entry points above): reads `bytes` bytes
 * (a multiple of 16) at `src` with 16-byte loads, non-temporal when
 * `nontemporal` is nonzero (the load type of the decode's K/V stream),
 * across a persistent grid, and computes nothing from them.  `sink` is a
 * 16-byte aligned 4-byte device word the kernel may write.  Its time per
 * call is the device's read rate for that many bytes.
 * ------------------------------------------------------------------------ */
int qwen3_hbm_read_reference(const void* src, int64_t bytes, int nontemporal, void* sink,
                             void* stream);

/* Matrix-core rate reference (no counterpart in the reference engine; for the
 * measurement of the prefill kernel): every wave of a persistent grid (two
 * 256-thread workgroups per CU) issues iters x 16 back-to-back
 * mfma_f32_32x32x16_bf16 products from registers, with no memory traffic.
 * *flops (host) receives the launch's flop count; `sink` is a 16-byte
 * aligned 4-byte device word the kernel may write.  Its time per call gives
 * the bf16 rate the device sustains, at the clock it holds under that load.
 * iters in [1, 2^24]. */
int qwen3_mfma_rate_reference(int iters, void* sink, int64_t* flops, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN3_ATTN_H */
