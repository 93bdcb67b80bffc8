/*
 * nie_paged.h — C ABI of the MI355X (gfx950) paged-attention library
 * (libnie_hip.so).
 *
 * The reference engine (ito-integral/nano-infer-engine) does this work with
 * PyTorch ATen ops called from Python loops.  Each entry point below replaces
 * one of those loops; the comment on each names the reference code it
 * replaces.  Paths are relative to the reference repository root.
 *
 * Conventions shared by every entry point
 *  - All data pointers are device pointers unless a comment says "host".
 *  - KV cache layout is the reference's storage layout, row-major
 *        keys/values : (num_layers, num_blocks, block_size, kv_heads, head_dim)
 *    (src/nano_infer_engine/paged_cache.py:71-79).  Offsets are computed in
 *    64-bit arithmetic, so pools larger than 2^31 elements are fine.
 *  - A "slot" is phys_block * block_size + offset_in_block
 *    (src/nano_infer_engine/paged_cache.py:240-262).
 *  - dtype is NIE_DTYPE_F32 or NIE_DTYPE_BF16; everything in one call shares it.
 *  - Attention shapes: q_heads a positive multiple of kv_heads and head_dim
 *    in [1, 256].  head_dim 64 or 128 with q_heads / kv_heads in
 *    {1, 2, 4, 8, 16} runs on the MFMA kernels, which need 16-byte aligned
 *    q/out/new-row pointers and strides; every other shape runs on a generic
 *    kernel (one wave per query row and head: the same results at a far
 *    lower rate), which needs element alignment only and no workspace (its
 *    *_workspace_bytes query returns 0).  block_size may be any positive
 *    value.
 *  - Block IDs read from block tables are clamped into [0, num_blocks) on the
 *    device, so a bad table cannot address memory outside the pool; callers
 *    validate tables on the host (the Python layer does).
 *  - Every call is asynchronous on `stream` (a hipStream_t; NULL = default
 *    stream).  The library never allocates or frees device memory: scratch
 *    space is the caller's `workspace`, sized by the *_workspace_bytes query.
 *    A decode or prefill workspace starts with a control region
 *    (nie_workspace_control_bytes()) that must be zero before the
 *    workspace's first call and that every call leaves zero; past it the
 *    workspace needs no initialisation.  Calls that overlap in time
 *    (different streams) need different workspaces.
 *  - Return value: NIE_OK, or a negative NIE_E* code; nie_last_error() then
 *    holds a message for the calling thread.
 */
#ifndef NIE_PAGED_H
#define NIE_PAGED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NIE_OK 0
#define NIE_EINVAL (-1)       /* bad argument (null pointer, bad size, bad workspace) */
#define NIE_EUNSUPPORTED (-2) /* dtype or shape not built (e.g. head_dim > 256) */
#define NIE_ELAUNCH (-3)      /* HIP reported an error at launch */

#define NIE_DTYPE_F32 0
#define NIE_DTYPE_BF16 1

/* Rounding point of the bf16 attention probabilities (nie_set_attention_rounding). */
#define NIE_ROUND_REFERENCE 0 /* the reference's: P = bf16(exp(s - m) / l), two passes over the keys */
#define NIE_ROUND_FAST 1      /* online softmax: bf16(exp(s - running max)), O / l at the end; one pass */

/* Library version string, e.g. "nie_paged 0.1 gfx950". */
const char* nie_version(void);

/* Message describing the last failed call made by this thread. */
const char* nie_last_error(void);

/*
 * KV append: scatter-writes the K and V rows of num_tokens new tokens into
 * one layer of the cache.  Token t goes to slot_mapping[t]; a negative slot
 * is skipped (padding), as is any slot >= num_blocks * block_size.
 *   k_new/v_new : (num_tokens, kv_heads, head_dim); token t starts at element
 *                 t * k_row_stride (resp. v_row_stride); heads and dims are
 *                 contiguous.
 * Bit-exact copy.
 * Replaces: the per-token copy loop of PagedKVCache.write
 *           (src/nano_infer_engine/paged_cache.py:264-322), called once per
 *           sequence by GroupedQueryAttention.forward
 *           (src/nano_infer_engine/layers/attention.py:246-253) and
 *           forward_ragged (attention.py:384-390).
 */
int nie_kv_append(int dtype,
                  const void* k_new, int64_t k_row_stride,
                  const void* v_new, int64_t v_row_stride,
                  const int64_t* slot_mapping, int64_t num_tokens,
                  void* k_cache, void* v_cache,
                  int64_t num_layers, int64_t layer_index,
                  int64_t num_blocks, int64_t block_size,
                  int64_t kv_heads, int64_t head_dim,
                  void* stream);

/*
 * KV gather: copies logical positions 0..token_count-1 of one sequence
 * (physical block table `block_table`, num_table_entries entries) into
 * contiguous (token_count, kv_heads, head_dim) tensors.  Bit-exact.
 * Replaces: the per-token gather loop + torch.stack of PagedKVCache.gather
 *           (src/nano_infer_engine/paged_cache.py:324-362).
 */
int nie_kv_gather(int dtype,
                  const void* k_cache, const void* v_cache,
                  int64_t num_layers, int64_t layer_index,
                  int64_t num_blocks, int64_t block_size,
                  int64_t kv_heads, int64_t head_dim,
                  const int32_t* block_table, int64_t num_table_entries,
                  int64_t token_count,
                  void* k_out, void* v_out,
                  void* stream);

/*
 * Block copy between two caches of identical (num_layers, block_size,
 * kv_heads, head_dim) geometry: for i < count, every layer of block
 * src_blocks[i] of the source pool is copied to block dst_blocks[i] of the
 * destination pool (both K and V).  Either side may instead be a packed
 * staging buffer of shape (num_layers, count, block_size, kv_heads, head_dim)
 * by passing a NULL block list for that side.  Bit-exact.
 * Replaces: the per-block torch.stack of PagedKVCache.export_sequence and the
 *           per-block copy_ of import_sequence
 *           (src/nano_infer_engine/paged_cache.py:145-238).
 */
int nie_kv_copy_blocks(int dtype,
                       const void* src_k, const void* src_v,
                       int64_t src_num_blocks, const int32_t* src_blocks,
                       void* dst_k, void* dst_v,
                       int64_t dst_num_blocks, const int32_t* dst_blocks,
                       int64_t count,
                       int64_t num_layers, int64_t block_size,
                       int64_t kv_heads, int64_t head_dim,
                       void* stream);

/*
 * Fused RoPE + KV append for num_tokens new tokens of one layer: rotates the
 * q rows in place, and writes the rotated k rows and the v rows to cache slot
 * slot_mapping[t] (a negative or out-of-pool slot skips the K/V write).
 *   q     : (num_tokens, q_heads, head_dim), element (t, h, d) at
 *           t * q_stride_t + h * q_stride_h + d;  k_new / v_new likewise
 *           with kv_heads heads.
 *   positions  : (num_tokens,) int64 absolute positions.
 *   cos_table / sin_table : (table_rows, head_dim / 2) in the storage dtype;
 *           row p holds cos / sin of p * inv_freq[i] (positions past the
 *           table are clamped to its last row; callers size the table).
 * Rotate-half with every product and sum rounded to the storage dtype, so
 * the output is bit-identical to the reference's elementwise torch ops fed
 * the same sin/cos rows; the K/V writes are bit-exact copies of those rows.
 * head_dim must be even (rotate-half splits it in two).
 * Replaces: the RoPE of q and k (src/nano_infer_engine/layers/rope.py:6-23,
 *           called at src/nano_infer_engine/layers/attention.py:238-239 and
 *           :375-376) followed by PagedKVCache.write of the new K/V
 *           (attention.py:246-253, :384-390; paged_cache.py:264-322).
 */
int nie_rope_kv_append(int dtype,
                       void* q, int64_t q_stride_t, int64_t q_stride_h, int64_t q_heads,
                       const void* k_new, int64_t k_stride_t, int64_t k_stride_h,
                       const void* v_new, int64_t v_stride_t, int64_t v_stride_h,
                       const int64_t* positions, const int64_t* slot_mapping, int64_t num_tokens,
                       const void* cos_table, const void* sin_table, int64_t table_rows,
                       void* k_cache, void* v_cache,
                       int64_t num_layers, int64_t layer_index,
                       int64_t num_blocks, int64_t block_size,
                       int64_t kv_heads, int64_t head_dim,
                       void* stream);

/*
 * RMSNorm of `rows` rows of `cols` elements: out = weight * (h / sqrt(mean(h*h)
 * + eps)) with h the row in fp32, the product in fp32 and the result rounded
 * to the storage dtype (weight NULL: no scale).  With residual != NULL the
 * row is first x + residual, rounded to the storage dtype and also written
 * to sum_out.  Rows are element strides apart; every row, the weight and
 * sum_out must be 16-byte aligned, and cols a multiple of 16 bytes' worth of
 * elements, at most 8192 (bf16) / 4096 (fp32).
 * Replaces: RmsNorm.forward (src/nano_infer_engine/layers/rms_norm.py:25-31)
 *           and, with residual, the residual add before the post-attention
 *           norm (src/nano_infer_engine/layers/decoder.py:50-51, :73-74).
 */
int nie_rms_norm(int dtype, const void* x, int64_t x_stride,
                 const void* residual, int64_t residual_stride,
                 void* sum_out, int64_t sum_stride,
                 const void* weight, void* out, int64_t out_stride,
                 int64_t rows, int64_t cols, float eps, void* stream);

/*
 * SwiGLU's gated product over rows x cols elements: out = silu(gate) * up,
 * silu(x) = x / (1 + exp(-x)) in fp32 rounded to the storage dtype, then the
 * product in fp32 rounded again (torch's two kernels).  Row r of each
 * operand starts at r * stride elements (gate and up may be the two halves
 * of one fused gate/up projection's output); rows 16-byte aligned and cols a
 * multiple of 16 bytes' worth of elements.
 * Replaces: F.silu(self.gate_proj(x)) * self.up_proj(x)
 *           (src/nano_infer_engine/layers/mlp.py:18-22).
 */
int nie_silu_mul(int dtype, const void* gate, int64_t gate_stride, const void* up, int64_t up_stride,
                 void* out, int64_t out_stride, int64_t rows, int64_t cols, void* stream);

/*
 * Projection GEMM of a decode step: y[m, j] = sum_i x[m, i] * w[j, i] for
 * m < rows, with w the (n, k) row-major weight of an nn.Linear (no bias),
 * bf16 operands, fp32 accumulation and one rounding to bf16.
 * epilogue NIE_LINEAR_SILU_MUL: w is the (2n, k) [gate; up] weight of a
 * SwiGLU block and y = silu(gate) * up over the n columns, with gate and up
 * rounded to bf16 first and nie_silu_mul's arithmetic after.
 * rows in 1..16, n a multiple of 16, k a multiple of 2048; x rows and w
 * 16-byte aligned; x_stride / y_stride are element strides between rows.
 * Other shapes return NIE_EUNSUPPORTED (callers then use a library GEMM).
 * Replaces, for decode steps: the nn.Linear projections of
 *           GroupedQueryAttention (q/k/v: src/nano_infer_engine/layers/attention.py:227-232,
 *           :359-361; o_proj: :271, :414), SwiGLUMLP's gate/up/down
 *           projections and their gated product
 *           (src/nano_infer_engine/layers/mlp.py:18-22) and the LM head
 *           (src/nano_infer_engine/models/llama.py:328, :391).
 */
#define NIE_LINEAR_PLAIN 0
#define NIE_LINEAR_SILU_MUL 1
int nie_linear_rows(int dtype, const void* x, int64_t x_stride, int64_t rows, const void* w, int64_t n,
                    int64_t k, int epilogue, void* y, int64_t y_stride, void* stream);

/*
 * nie_linear_rows with the RMSNorm that precedes the projection folded into
 * its x operand: h = x (+ residual, rounded to bf16), then
 * y = epilogue(norm(h) . w^T) with norm(h) = norm_weight * (h / sqrt(mean(h*h)
 * + eps)) rounded to bf16 — nie_rms_norm's arithmetic (only the order of
 * the sum of squares differs).  With residual and sum_out, h is also written
 * to sum_out (rows of k elements, sum_stride apart).  k must be 2048;
 * norm_weight (k elements) is required; residual and sum_out may be NULL
 * (sum_out needs residual).  Other arguments as nie_linear_rows.
 * Replaces, for decode steps: RmsNorm.forward (src/nano_infer_engine/layers/rms_norm.py:25-31)
 *           with the residual add before it (src/nano_infer_engine/layers/decoder.py:50-51)
 *           followed by the q/k/v, gate/up or LM-head projection
 *           (src/nano_infer_engine/layers/attention.py:227-232,
 *           src/nano_infer_engine/layers/mlp.py:18-22,
 *           src/nano_infer_engine/models/llama.py:328).
 */
int nie_rms_norm_linear_rows(int dtype, const void* x, int64_t x_stride, const void* residual,
                             int64_t residual_stride, void* sum_out, int64_t sum_stride,
                             const void* norm_weight, float eps, int64_t rows, const void* w, int64_t n,
                             int64_t k, int epilogue, void* y, int64_t y_stride, void* stream);

/*
 * Greedy token selection: out[r] = index of the largest of the cols values
 * of row r (element (r, c) at r * row_stride + c), ties to the lowest index,
 * NaN larger than every number — torch.argmax's result.  out is int64.
 * Replaces: torch.stack(request_logits).argmax(dim=-1) of the scheduler step
 *           (src/nano_infer_engine/generation/scheduler.py:399-401), here
 *           run on the logits rows as the step's last kernel so a captured
 *           decode step ends with the next token IDs on the device.
 */
int nie_argmax_rows(int dtype, const void* logits, int64_t rows, int64_t cols, int64_t row_stride,
                    int64_t* out, void* stream);

/*
 * nie_argmax_rows for long rows: one workgroup per piece of 8192 columns of
 * a row, then a merge of the pieces' (value, index) pairs; the result is
 * nie_argmax_rows's (the comparison is a strict total order).  workspace:
 * device memory of nie_argmax_rows_workspace_bytes(rows, cols) bytes,
 * 16-byte aligned, no initialisation needed; calls that overlap in time need
 * different workspaces.
 * Replaces: as nie_argmax_rows (src/nano_infer_engine/generation/scheduler.py:399-401),
 *           for LM-head rows of 128256 logits.
 */
int64_t nie_argmax_rows_workspace_bytes(int64_t rows, int64_t cols);
int nie_argmax_rows_split(int dtype, const void* logits, int64_t rows, int64_t cols, int64_t row_stride,
                          int64_t* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Where the bf16 attention kernels (nie_paged_decode*, nie_varlen_prefill)
 * round the softmax probabilities, for calls issued after this one in the
 * whole process (default NIE_ROUND_REFERENCE).
 *  NIE_ROUND_REFERENCE: the reference's rounding point.  Scores are
 *    bf16(bf16(q.k) * scale), the softmax runs in fp32 over a row's whole
 *    key range, the normalised probabilities exp(s - m) / l are rounded to
 *    bf16, and P.V accumulates them in fp32 (rounded once).  The kernels make
 *    two passes over the keys: the first forms each row's maximum and sum
 *    (decode: and keeps every score in the workspace), the second the
 *    probabilities and P.V.
 *  NIE_ROUND_FAST: one pass with an online softmax; the unnormalised
 *    exp(s - running maximum) is rounded to bf16 and the row is divided by
 *    its sum at the end (flash-attention style).  Same inputs to the softmax,
 *    a different rounding point for P.
 * fp32 calls are unaffected (the probabilities are not rounded).  The
 * workspace sizes depend on the mode: query them after setting it.
 * NIE_EINVAL for any other value.
 * Replaces: the probability cast of the reference's softmax
 *           (src/nano_infer_engine/layers/paged_attention.py:109-114,
 *           layers/attention.py:410-411), which the default mode keeps.
 */
int nie_set_attention_rounding(int mode);
int nie_attention_rounding(void);

/*
 * The one-launch reference-rounding decode.  With the reference rounding, a
 * bf16 decode call whose head_dim is 64, whose block_size is a power of two
 * of at least 16, whose GQA group has at most 4 query heads and whose work
 * items can all be resident on the GPU at once runs as one kernel instead of
 * the two pass launches and the sum of their split partials: each split
 * keeps its scores on chip, the splits exchange only their (max, sum) pairs
 * and output shares, through counters in the workspace's control region,
 * and the split that finishes last sums the shares.  nie_set_decode_fused(0)
 * turns it off for calls issued after it in the whole process (1, the
 * default, on); the pass launches then run the same plan, so both give the
 * same bits.  The switch also covers the one-pass rounding (fp32, and bf16
 * with NIE_ROUND_FAST): there, when a call splits its sequences' keys, the
 * split of a (sequence, KV head) that finishes last merges the split
 * partials inside the decode kernel (a counter per pair in the control
 * region, up to 2047 pairs) instead of a separate merge launch, in the
 * merge launch's order (the same bits), in calls of at most a quarter of
 * the CUs' workgroups (larger calls keep the merge launch, which costs them
 * less); 2 does so in calls of every size (as 1 otherwise).  NIE_EINVAL for
 * other values.
 * No counterpart in the reference (an execution strategy of its decode
 * attention, layers/paged_attention.py:88-116).
 */
int nie_set_decode_fused(int on);
int nie_decode_fused(void);

/*
 * Polls a split of the one-launch decode makes, waiting for the other
 * splits of its sequence, before it forms their (max, sum) pairs itself
 * from K (the same numbers, at the cost of reading their keys); default
 * 32768.  0 makes every wait give up at once, which tests use to run that
 * path.  NIE_EINVAL for negative values.
 * No counterpart in the reference.
 */
int nie_set_decode_fused_spin(int polls);

/*
 * Bytes at the start of every decode and prefill workspace that hold the
 * control region (counters of the one-launch decode).  They must be zero
 * before a workspace is first used; every call leaves its counters zero, so
 * a workspace needs clearing only once, when it is allocated.  The
 * workspace queries include these bytes.
 * No counterpart in the reference.
 */
int64_t nie_workspace_control_bytes(void);

/* Which kernels the calling thread's last nie_paged_decode* call ran. */
#define NIE_DECODE_PATH_NONE 0     /* no call yet, or it failed before launching */
#define NIE_DECODE_PATH_ONE_PASS 1 /* fp32, or bf16 with NIE_ROUND_FAST (merge launch when split) */
#define NIE_DECODE_PATH_PASSES 2   /* reference rounding: scores pass, P.V pass, sum */
#define NIE_DECODE_PATH_FUSED 3    /* reference rounding: the one-launch decode, sum */
#define NIE_DECODE_PATH_GENERIC 4  /* shapes outside the MFMA kernels */
#define NIE_DECODE_PATH_ONE_PASS_MERGED 5 /* one pass, split, merged by the last split: one launch */
int nie_decode_last_path(void);

/*
 * Workspace bytes needed by nie_paged_decode for a call with these
 * arguments (same meaning as there; host values), whose sequence lengths
 * have maximum max_seq_len and sum total_seq_len, and the same optional
 * host copy of the lengths as the call.  The split of the work depends on
 * all of them, so query with the values of the call.
 * Layout: the control region (nie_workspace_control_bytes(); zero before
 * the workspace's first call, left zero by every call), then fp32 split
 * partials (O rows, then (max, sum) pairs); with the reference rounding
 * (bf16) also the bf16 scores of every key of the call.  The pointer must
 * be 16-byte aligned.  Returns 0 for invalid arguments.
 */
int64_t nie_paged_decode_workspace_bytes(int dtype, int64_t batch, int64_t q_heads,
                                         int64_t kv_heads, int64_t head_dim,
                                         int64_t block_size, int64_t max_seq_len,
                                         int64_t total_seq_len,
                                         const int32_t* host_seq_lens);

/*
 * Paged decode attention: one query token per sequence attends to the first
 * seq_lens[b] cached tokens of its sequence (no causal mask needed: the
 * current token is already cached).  GQA: query head h reads KV head
 * h / (q_heads / kv_heads).
 *   q     : (batch, q_heads, head_dim), element (b, h, d) at
 *           b * q_stride_b + h * q_stride_h + d.
 *   out   : same indexing with out_stride_b / out_stride_h.
 *   block_tables : (batch, table_stride) int32, row b = physical blocks of
 *           sequence b in logical order.
 *   seq_lens     : (batch,) int32 device copy of the lengths, each >= 1.
 *   max_seq_len / total_seq_len : host copies of max and sum of seq_lens;
 *           they size the launch and must be exact.
 *   host_seq_lens : optional HOST copy of seq_lens (NULL: none).  With it the
 *           launch is planned from the exact lengths (split length chosen so
 *           the work fills the GPU's resident workgroups, every workgroup a
 *           real work item), and the work items are passed to the kernels in
 *           their arguments.  It must hold the same values as seq_lens;
 *           NIE_EINVAL if it does not match max_seq_len / total_seq_len.
 * Long sequences are split over several workgroups whose fp32 partials a
 * second kernel, on the same stream, merges exactly (log-sum-exp weights).
 * Numerics follow the reference: the q.k score is rounded to the storage
 * dtype and scaled in that dtype, softmax runs in fp32, P.V accumulates in
 * fp32 and the result is rounded to the storage dtype.
 * Replaces: paged_attention_reference / batched_paged_attention_reference
 *           (src/nano_infer_engine/layers/paged_attention.py:4-176), called
 *           from GroupedQueryAttention.forward
 *           (src/nano_infer_engine/layers/attention.py:255-269), and the
 *           length-1 rows of forward_ragged (attention.py:380-412).
 */
int nie_paged_decode(int dtype,
                     const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache,
                     int64_t num_layers, int64_t layer_index,
                     int64_t num_blocks, int64_t block_size,
                     int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                     const int32_t* block_tables, int64_t table_stride,
                     const int32_t* seq_lens, int64_t batch,
                     int64_t max_seq_len, int64_t total_seq_len,
                     float scale,
                     void* out, int64_t out_stride_b, int64_t out_stride_h,
                     void* workspace, int64_t workspace_bytes,
                     const int32_t* host_seq_lens,
                     void* stream);

/*
 * Decode step with the cache update in the same launch: for each sequence b
 * it writes the new key/value rows k_new[b] / v_new[b] (kv_heads x head_dim,
 * heads contiguous; row strides k_new_stride / v_new_stride elements) at
 * logical position seq_lens[b] - 1, in the slot its block table gives
 * (block_tables[b][p / block_size] * block_size + p % block_size), then
 * attends over positions [0, seq_lens[b]) exactly as nie_paged_decode.  The
 * cache and the output equal those of nie_kv_append with that slot mapping
 * followed by nie_paged_decode, provided no other sequence of the call reads
 * that slot (the block of a sequence's newest token is its own).  A table
 * entry outside [0, num_blocks) skips the write, as an out-of-range slot
 * skips nie_kv_append.  Workspace: nie_paged_decode_workspace_bytes.
 * With cos_table / sin_table ((table_rows, head_dim / 2) in the storage
 * dtype; NULL: none), q and the new K rows are first rotated at position
 * seq_lens[b] - 1 exactly as nie_rope_kv_append rotates them (q is not
 * written back), so the call equals nie_rope_kv_append then
 * nie_paged_decode on a decode-only batch.
 * Replaces: the decode step of GroupedQueryAttention.forward's paged branch
 *           (src/nano_infer_engine/layers/attention.py:246-269): one
 *           PagedKVCache.write per sequence at its cached length
 *           (paged_cache.py:264-322), then batched_paged_attention_reference
 *           with lengths + 1; with the tables also the RoPE of q and k before
 *           it (attention.py:238-239, layers/rope.py:171-200).
 */
int nie_paged_decode_append(int dtype,
                            const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const void* k_new, int64_t k_new_stride,
                            const void* v_new, int64_t v_new_stride,
                            const void* cos_table, const void* sin_table, int64_t table_rows,
                            void* k_cache, void* v_cache,
                            int64_t num_layers, int64_t layer_index,
                            int64_t num_blocks, int64_t block_size,
                            int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            const int32_t* block_tables, int64_t table_stride,
                            const int32_t* seq_lens, int64_t batch,
                            int64_t max_seq_len, int64_t total_seq_len,
                            float scale,
                            void* out, int64_t out_stride_b, int64_t out_stride_h,
                            void* workspace, int64_t workspace_bytes,
                            const int32_t* host_seq_lens,
                            void* stream);

/*
 * A decode plan in memory, for launches captured once and replayed with
 * other lengths (a HIP graph of the decode step).  nie_paged_decode_plan
 * writes into `plan` (nie_paged_decode_plan_bytes() bytes, 4-byte aligned,
 * host memory) the work items nie_paged_decode_append would plan from
 * host_seq_lens (the same values as the device lengths of the launch it is
 * for; each in [1, max_seq_len], reaching max_seq_len, summing to
 * total_seq_len) for these shapes; the caller copies the bytes to device
 * memory.  nie_paged_decode_append_planned is nie_paged_decode_append
 * planned from bounds (max_seq_len, total_seq_len as upper bounds; its
 * workspace nie_paged_decode_workspace_bytes of those bounds, its kernel
 * arguments fixed), whose kernels take their work items from device_plan at
 * run time when the table there has any (a table of count 0, as written for
 * shapes the MFMA kernels do not take or for more items or sequences than a
 * table holds, leaves them to locate their work from the device lengths).
 * With a table, its result is bit-identical to nie_paged_decode_append
 * called with those host lengths; without one (count 0, split length 0),
 * to nie_paged_decode_append planned from the same bounds.  No counterpart in the reference (whose
 * decode step runs eagerly, docs/development-roadmap.md:89, :190 list graph
 * capture as future work); it exists for replayed decode steps, which
 * cannot pass host lengths in kernel arguments.
 */
int64_t nie_paged_decode_plan_bytes(void);
int nie_paged_decode_plan(int dtype, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                          int64_t block_size, const int32_t* host_seq_lens, int64_t batch,
                          int64_t max_seq_len, int64_t total_seq_len, void* plan, int64_t plan_bytes);
int nie_paged_decode_append_planned(int dtype,
                                    const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    const void* k_new, int64_t k_new_stride,
                                    const void* v_new, int64_t v_new_stride,
                                    const void* cos_table, const void* sin_table, int64_t table_rows,
                                    void* k_cache, void* v_cache,
                                    int64_t num_layers, int64_t layer_index,
                                    int64_t num_blocks, int64_t block_size,
                                    int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                    const int32_t* block_tables, int64_t table_stride,
                                    const int32_t* seq_lens, int64_t batch,
                                    int64_t max_seq_len, int64_t total_seq_len,
                                    float scale,
                                    void* out, int64_t out_stride_b, int64_t out_stride_h,
                                    void* workspace, int64_t workspace_bytes,
                                    const void* device_plan,
                                    void* stream);

/*
 * nie_paged_decode_append without a workspace argument: the split partials
 * go to a device array the library owns (nie_paged_decode_noalloc_max_bytes()
 * bytes = 32 MiB per GPU, held from the device's first call until the
 * process ends).  The call allocates nothing (no hipMalloc, no allocating
 * library routine); the first call on a device looks the array's address up
 * once.  Every other argument, and the result, is nie_paged_decode_append's.
 * A call whose partials would exceed the array (nie_paged_decode_workspace_bytes
 * of the same arguments above the maximum, for a call that splits) returns
 * NIE_EINVAL with a message saying so.  All calls on one GPU share the
 * array: calls that overlap in time on one GPU (different streams, or
 * different threads) race.  Nothing in the array needs clearing between
 * calls (each call writes every partial it reads).
 * No counterpart in the reference: this entry point exists for callers that
 * cannot allocate device memory — code under HIP graph capture, tight
 * serving loops and harnesses that forbid hipMalloc.
 */
int64_t nie_paged_decode_noalloc_max_bytes(void);
int nie_paged_decode_append_noalloc(int dtype,
                                    const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    const void* k_new, int64_t k_new_stride,
                                    const void* v_new, int64_t v_new_stride,
                                    const void* cos_table, const void* sin_table, int64_t table_rows,
                                    void* k_cache, void* v_cache,
                                    int64_t num_layers, int64_t layer_index,
                                    int64_t num_blocks, int64_t block_size,
                                    int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                    const int32_t* block_tables, int64_t table_stride,
                                    const int32_t* seq_lens, int64_t batch,
                                    int64_t max_seq_len, int64_t total_seq_len,
                                    float scale,
                                    void* out, int64_t out_stride_b, int64_t out_stride_h,
                                    const int32_t* host_seq_lens,
                                    void* stream);

/*
 * Workspace bytes needed by nie_varlen_prefill (host values: number of
 * sequences, total and maximum query length, maximum context+query length,
 * and the same optional host copies of cu_seqlens_q / context_lens as the
 * call, which change the launch plan).  Returns 0 when no workspace is
 * needed or the arguments are invalid.  A workspace starts with the
 * control region (nie_workspace_control_bytes(), which prefill leaves
 * alone), so one buffer can serve decode and prefill calls in turn.
 */
int64_t nie_varlen_prefill_workspace_bytes(int64_t num_seqs, int64_t total_query_tokens,
                                           int64_t max_query_len, int64_t max_seq_len,
                                           int64_t q_heads, int64_t kv_heads,
                                           int64_t head_dim,
                                           const int64_t* host_cu_seqlens,
                                           const int32_t* host_context_lens);

/*
 * Varlen (chunked-prefill) attention over the paged cache.  Sequence r owns
 * packed query rows cu_seqlens_q[r] .. cu_seqlens_q[r+1]-1; row i of it sits
 * at absolute position context_lens[r] + i and attends to cached positions
 * 0 .. that position (causal inside the chunk, full attention to the prior
 * context).  The chunk's own K/V must already be in the cache.
 *   q   : (total_query_tokens, q_heads, head_dim), element (t, h, d) at
 *         t * q_stride_t + h * q_stride_h + d;  out likewise.
 *   cu_seqlens_q : (num_seqs + 1,) int64, cu_seqlens_q[0] == 0.
 *   context_lens : (num_seqs,) int32.
 *   total_query_tokens, max_query_len, max_seq_len: host values sizing the
 *         launch; they must be exact (max_seq_len = max of context + query).
 *   host_cu_seqlens / host_context_lens: optional (both or neither) HOST
 *         copies of cu_seqlens_q / context_lens.  With them the launch is
 *         planned from the exact work: key splits sized so the work fills
 *         the GPU about once, and a grid of exactly the work items.  Without
 *         them the plan uses upper bounds from the sizes above.  They must
 *         hold the same values as the device arrays; NIE_EINVAL if they do
 *         not fit the sizes.
 * Query tiles whose keys are split over several workgroups are merged
 * exactly (log-sum-exp weights) by a second kernel on the same stream.
 * Numerics as nie_paged_decode.
 * Replaces: the per-request write/gather/repeat_interleave/matmul/mask/
 *           softmax/matmul loop of GroupedQueryAttention.forward_ragged
 *           (src/nano_infer_engine/layers/attention.py:378-414) and the dense
 *           attention of the non-chunked paged prefill
 *           (src/nano_infer_engine/models/llama.py:274-325).
 */
int nie_varlen_prefill(int dtype,
                       const void* q, int64_t q_stride_t, int64_t q_stride_h,
                       const int64_t* cu_seqlens_q, const int32_t* context_lens,
                       int64_t num_seqs, int64_t total_query_tokens,
                       int64_t max_query_len, int64_t max_seq_len,
                       const void* k_cache, const void* v_cache,
                       int64_t num_layers, int64_t layer_index,
                       int64_t num_blocks, int64_t block_size,
                       int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                       const int32_t* block_tables, int64_t table_stride,
                       float scale,
                       void* out, int64_t out_stride_t, int64_t out_stride_h,
                       void* workspace, int64_t workspace_bytes,
                       const int64_t* host_cu_seqlens, const int32_t* host_context_lens,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NIE_PAGED_H */
