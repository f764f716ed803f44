/*
 * voom_hip.h - C ABI of libvoom_hip.so, the MI355X (gfx950) kernels behind the
 * paged-KV path: paged GQA decode attention, absorbed-MLA latent decode, the
 * byte-plane spill codec and the page append/gather/scatter helpers.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise.  The
 *     caller owns all memory (PyTorch tensors in the Python host layer).
 *   - bf16 data is passed as raw 16-bit words (uint16_t bit patterns).
 *   - Every entry point takes a hipStream_t (NULL = legacy default stream) and
 *     only enqueues work; nothing synchronises.
 *   - Return value: 0 on success; VOOM_EINVAL (negative) when an argument fails
 *     validation; a positive hipError_t when a HIP call or launch fails.
 *     voom_last_error() returns a thread-local message for the last failure.
 *
 * Device page layouts (one tensor per layer)
 *   K pool  [num_slots, num_kv_heads, page_tokens, head_dim]   token-major
 *   V pool  [num_slots, num_kv_heads, page_tokens/VB, head_dim, VB]
 *           V^T in blocks of VB = min(page_tokens, 32) tokens
 *   latent  [num_slots, page_tokens, latent_dim]               token-major
 *   block_table [batch, max_pages] int32 slot ids, ctx_lens [batch] int32.
 *   V is stored as transposed 32-token blocks so that the P.V contraction
 *   reads 16 contiguous bytes per lane straight into the MFMA operand and each
 *   block of K and of V is one contiguous run (64 * head_dim bytes).
 */
#ifndef VOOM_HIP_H
#define VOOM_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VOOM_OK 0
#define VOOM_EINVAL (-1)

/* Thread-local message describing the last non-zero return. */
const char* voom_last_error(void);

/* ABI version, bumped on any signature or layout change (2: checksums in the
 * slot codec; 3: spill-record calls; 4: element and table types of the
 * position-free call; 5: the top-k workspace's zeroed row counters; 6:
 * voom_copy_rows). */
int voom_abi_version(void);

/* ---------------------------------------------------------------------------
 * Paged GQA decode attention (one query token per sequence).
 *
 * Replaces the decode attention of the reference: PagedKVCache.update
 * concatenating every page (runtime/kv_paged.py:164-181) followed by
 * mx.fast.scaled_dot_product_attention(q, K, V, scale=hd**-0.5) with the GQA
 * broadcast inside SDPA (runtime/layer_runner.py:158,179-180), and the
 * page-table-indirect Metal kernel position_free_paged_attention
 * (runtime/pic_attention.py:184-232, page index ((blk*NKV+kvh)*BLOCK+off)*D).
 *
 *   q        [batch, num_q_heads, head_dim] bf16 (already RoPE-rotated)
 *   out      [batch, num_q_heads, head_dim] bf16
 *   lse_out  [batch, num_q_heads] fp32 natural-log sum-exp of the scaled
 *            scores, or NULL.  Lets two calls over disjoint page sets be merged
 *            with voom_merge_attn_states.
 *   num_splits  number of wavefronts sharing the work (0 = library choice:
 *            a block table of at most 1024 tokens per sequence then runs one
 *            workgroup per (sequence, kv head) that merges its own waves and
 *            writes out directly -- one launch, workspace untouched; longer
 *            tables split-K over the default count); the workspace must hold
 *            voom_paged_gqa_workspace_bytes(...) bytes for the same value.
 * head_dim in {64, 128}; num_q_heads / num_kv_heads <= 16; page_tokens a power
 * of two >= 32.  Sequences with ctx_len 0 produce zeros (lse = -inf).
 * ------------------------------------------------------------------------- */
size_t voom_paged_gqa_workspace_bytes(int batch, int num_q_heads, int num_kv_heads,
                                      int head_dim, int num_splits);
int voom_paged_gqa_default_splits(void);
int voom_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                          const int32_t* block_table, const int32_t* ctx_lens,
                          void* out, float* lse_out, void* workspace, size_t ws_bytes,
                          int batch, int num_q_heads, int num_kv_heads, int head_dim,
                          int page_tokens, int max_pages, int num_slots, float scale,
                          int num_splits, hipStream_t stream);

/* voom_paged_gqa_decode without a workspace: the split partials live in a
 * file-scope device array of voom_paged_gqa_noalloc_max_bytes() bytes (16 MiB)
 * held by each device for the life of the process, so the call allocates
 * nothing.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * voom_paged_gqa_decode minus the workspace; a request whose partials exceed
 * the array fails with VOOM_EINVAL.  The stream must belong to the current
 * device.  Calls that overlap on one device share the array and race. */
size_t voom_paged_gqa_noalloc_max_bytes(void);
int voom_paged_gqa_decode_noalloc(const void* q, const void* k_pool, const void* v_pool,
                                  const int32_t* block_table, const int32_t* ctx_lens,
                                  void* out, float* lse_out, int batch, int num_q_heads,
                                  int num_kv_heads, int head_dim, int page_tokens,
                                  int max_pages, int num_slots, float scale, int num_splits,
                                  hipStream_t stream);

/* The two halves of voom_paged_gqa_decode, for callers that time or schedule
 * them separately (same arguments, same workspace, same num_splits):
 *   voom_paged_gqa_partials  streams the pages once and leaves one partial
 *                            softmax state (m, l, o) per split piece in the
 *                            workspace (the main, HBM-bound kernel);
 *   voom_paged_gqa_combine   merges each head's partial states into out and
 *                            lse_out (the online-softmax merge of
 *                            runtime/pic_attention.py:106-129).
 * voom_paged_gqa_decode(...) with num_splits > 0, or a table longer than 1024
 * tokens, is exactly partials followed by combine. */
int voom_paged_gqa_partials(const void* q, const void* k_pool, const void* v_pool,
                            const int32_t* block_table, const int32_t* ctx_lens,
                            void* workspace, size_t ws_bytes, int batch, int num_q_heads,
                            int num_kv_heads, int head_dim, int page_tokens, int max_pages,
                            int num_slots, float scale, int num_splits, hipStream_t stream);
int voom_paged_gqa_combine(const int32_t* ctx_lens, void* out, float* lse_out,
                           void* workspace, size_t ws_bytes, int batch, int num_q_heads,
                           int num_kv_heads, int head_dim, int page_tokens, int max_pages,
                           int num_splits, hipStream_t stream);

/* Merge two attention states over disjoint key sets (log-sum-exp combine):
 * out = (o_a*e^{lse_a} + o_b*e^{lse_b}) / (e^{lse_a} + e^{lse_b}).
 * o_a/o_b/out [rows, head_dim] bf16, lse_* [rows] fp32; lse_out may be NULL.
 * Replaces the running (max, sum, acc) merge of the reference's online key
 * tiles (runtime/glm.py:165-196) and the simdgroup merge of the Metal kernel
 * (runtime/pic_attention.py:106-129). */
int voom_merge_attn_states(const void* o_a, const float* lse_a, const void* o_b,
                           const float* lse_b, void* out, float* lse_out, int rows,
                           int head_dim, hipStream_t stream);

/* Fold a bf16 attention state (o_b [rows, head_dim], lse_b [rows]) over a key
 * set disjoint from the accumulator's into an fp32 running state (o_acc
 * [rows, head_dim], lse_acc [rows]) in place; init != 0 sets the state to
 * (o_b, lse_b).  The running output stays fp32 across any number of folds
 * (rounded once by the caller), as the reference's online key tiles keep fp32
 * (max, sum, acc) across tiles (runtime/glm.py:165-196). */
int voom_fold_attn_state(float* o_acc, float* lse_acc, const void* o_b, const float* lse_b,
                         int rows, int head_dim, int init, hipStream_t stream);

/* voom_mla_head_gemv: y[b, h, n] = bf16(sum_k x[b, h, k] w[h, k, n]), fp32
 * sums, for the few query rows of a decode step -- the absorption products
 * q_nope . W_UK (runtime/glm.py:129-132) and weighted_c . W_UV
 * (runtime/glm.py:200-202) that the reference runs as batched products with
 * M = batch.  x [batch, num_heads, x_stride] (first k used), w_packed from
 * voom_mla_pack_head_weights for the same (num_heads, k, n), y [batch,
 * num_heads, y_stride] (first n written); batch 1..16, any k, n >= 1. */
int voom_mla_head_gemv(const void* x, const void* w_packed, void* y, int batch, int num_heads,
                       int k, int n, int x_stride, int y_stride, hipStream_t stream);

/* voom_mla_absorb_query: q_lat [batch, num_heads, c_dim + rope_dim] =
 * [q_nope . W_UK | q_rope] in one launch (runtime/glm.py:129-132): q_nope
 * [batch, num_heads, dn], q_rope [batch, num_heads, rope_dim], w_uk_packed
 * = W_UK [num_heads, dn, c_dim] packed by voom_mla_pack_head_weights. */
int voom_mla_absorb_query(const void* q_nope, const void* q_rope, const void* w_uk_packed,
                          void* q_lat, int batch, int num_heads, int dn, int c_dim, int rope_dim,
                          hipStream_t stream);

/* Bytes of the packed form of per-head weights w [num_heads, k, n] bf16
 * (k and n padded to multiples of 32 and 16). */
size_t voom_mla_head_weights_bytes(int num_heads, int k, int n);

/* Pack w [num_heads, k, n] bf16 into w_packed (voom_mla_head_weights_bytes,
 * 16-byte aligned) in the operand order of voom_mla_head_gemv's matrix
 * instructions; done once per weight matrix (the reference keeps W_UK and
 * W_UV as slices of kv_b_proj, runtime/glm.py:124-125). */
int voom_mla_pack_head_weights(const void* w, void* w_packed, int num_heads, int k, int n,
                               hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Absorbed-MLA paged decode: the latent contraction.
 *
 * Replaces the latent part of _mla_absorbed_attention (runtime/glm.py:133-164):
 * scores = q_lat . lat^T * scale in fp32, softmax, probabilities rounded to
 * bf16, weighted_c = p . lat[:, :512] returned in bf16.  The latent cache is
 * paged: lat_pool [num_slots, page_tokens, latent_dim] bf16, one slot holding
 * page_tokens consecutive tokens of one sequence (the compressed cache of
 * glm.py:265-274 / kv_cache.py:99-105, paged).
 *   q_lat  [batch, num_heads, latent_dim] bf16 = [q_nope . W_UK | q_rope]
 *   out_c  [batch, num_heads, c_dim] bf16 (weighted_c)
 *   lse_out [batch, num_heads] fp32 natural-log sum-exp, or NULL
 * latent_dim 576 with c_dim 512 (kv_lora_rank 512 + rope 64); num_heads a
 * multiple of 32; page_tokens a power of two >= 64.  num_ranges splits each
 * sequence's tokens (0 = library default); the workspace must hold
 * voom_mla_workspace_bytes(batch, num_heads, num_ranges) bytes.
 * ------------------------------------------------------------------------- */
size_t voom_mla_workspace_bytes(int batch, int num_heads, int num_ranges);
int voom_mla_absorbed_decode(const void* q_lat, const void* lat_pool,
                             const int32_t* block_table, const int32_t* ctx_lens,
                             void* out_c, float* lse_out, void* workspace, size_t ws_bytes,
                             int batch, int num_heads, int latent_dim, int c_dim,
                             int page_tokens, int max_pages, int num_slots, float scale,
                             int num_ranges, hipStream_t stream);

/* voom_mla_absorbed_decode_project: voom_mla_absorbed_decode followed by the
 * output projection y [batch, num_heads, dv] = weighted_c . W_UV
 * (runtime/glm.py:200-202), the merge of the range partials and the
 * projection in one launch; num_heads a multiple of 64, batch <= 16, dv <=
 * 128, w_uv_packed = W_UV^T [num_heads, c_dim, dv] packed by
 * voom_mla_pack_head_weights.  wc_out [batch, num_heads, c_dim] (weighted_c,
 * bf16) and lse_out are optional (null). */
int voom_mla_absorbed_decode_project(const void* q_lat, const void* lat_pool,
                                     const int32_t* block_table, const int32_t* ctx_lens,
                                     const void* w_uv_packed, int dv, void* y, void* wc_out,
                                     float* lse_out, void* workspace, size_t ws_bytes, int batch,
                                     int num_heads, int latent_dim, int c_dim, int page_tokens,
                                     int max_pages, int num_slots, float scale, int num_ranges,
                                     hipStream_t stream);

/* The same contraction over a selection of each sequence's positions: the
 * DSA gather of the top-k latent rows feeding absorbed MLA
 * (runtime/glm.py:280-289).  sel [batch, sel_stride] int32 holds ascending
 * logical positions (voom_dsa_topk's output), sel_lens [batch] how many are
 * used; the rows are read through block_table straight from the pool (no
 * gathered copy).  The pool must be smaller than 4 GiB.  num_ranges 0 picks
 * a split sized to the selection; the workspace must hold
 * voom_mla_sparse_workspace_bytes(batch, num_heads, sel_stride, num_ranges). */
size_t voom_mla_sparse_workspace_bytes(int batch, int num_heads, int sel_stride, int num_ranges);
int voom_mla_sparse_decode(const void* q_lat, const void* lat_pool, const int32_t* block_table,
                           const int32_t* sel, const int32_t* sel_lens, void* out_c,
                           float* lse_out, void* workspace, size_t ws_bytes, int batch,
                           int num_heads, int latent_dim, int c_dim, int page_tokens,
                           int max_pages, int num_slots, int sel_stride, float scale,
                           int num_ranges, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * DSA (DeepSeek Sparse Attention) selection for a decode step.
 *
 * voom_dsa_index_scores replaces the lightning-indexer scores of
 * DSAState.update_and_select (runtime/glm_dsa.py:140-150):
 *   scores[b][s] = sum_j w_head[b][j] * max(scale * (q_idx[b][j] . k_idx[b][s]), 0)
 * in fp32 for s < lens[b].  q_idx [batch, num_heads, head_dim] bf16 (after the
 * indexer RoPE), w_head [batch, num_heads] fp32 (weights_proj output already
 * multiplied by num_heads^-0.5), k_idx [batch, cap, head_dim] bf16 (the
 * cached index keys), scores [batch, cap] fp32 (entries at or past lens[b]
 * are not written).  head_dim 128; num_heads 16, 32, 48 or 64.
 *
 * voom_dsa_topk replaces the selection (glm_dsa.py:151-160): the k highest
 * scores of keys s < lens[b] (causal for a decode step at position
 * lens[b] - 1), written to sel [batch, k] as ascending indices, with
 * sel_lens[b] = min(lens[b], k).  Among keys tied at the k-th score the
 * lowest indices are kept.  One launch.  The workspace (candidate slots and
 * one arrival counter per row) must hold voom_dsa_topk_workspace_bytes(batch,
 * cap) bytes, and its first 4 * batch bytes must be zero before the first
 * call (allocate it zeroed); every call leaves them zero again.  Calls that
 * share a workspace must not overlap.
 * ------------------------------------------------------------------------- */
int voom_dsa_index_scores(const void* q_idx, const float* w_head, const void* k_idx,
                          const int32_t* lens, float* scores, int batch, int num_heads,
                          int head_dim, int cap, float scale, hipStream_t stream);
size_t voom_dsa_topk_workspace_bytes(int batch, int cap);
int voom_dsa_topk(const float* scores, const int32_t* lens, int32_t* sel, int32_t* sel_lens,
                  void* workspace, size_t ws_bytes, int batch, int cap, int k,
                  hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Position-free paged attention (keys stored before RoPE).
 *
 * Replaces position_free_paged_attention and its Metal kernel
 * (runtime/pic_attention.py:22-232), with the same accepted inputs: pages
 * hold unrotated K and ordinary V, [num_pages, num_kv_heads, block_size,
 * head_dim] each; block_table [ceil(num_keys / block_size)] int32 maps the
 * logical keys (shared by all batch rows; repeating a page id is legal and is
 * how pages are shared); key k is rotated at key_positions[k] with the NeoX
 * tables cos/sin [max_position, head_dim/2] in fp32, rounded to the element
 * type, and attended by query tq iff key_positions[k] <= query_positions[tq].
 *   q    [batch, num_q_heads, num_queries, head_dim], already rotated
 *   out  same shape; rows with no visible key are zeros
 * dtype: the element type of q, the pages and out (VOOM_DTYPE_BF16, _F16 or
 * _F32; the reference's T).  table_dtype: VOOM_DTYPE_F32 or dtype (the
 * reference's "FP32 or match the Q/K/V dtype", :210-211).  head_dim a
 * multiple of 32 up to 256 (the reference: any multiple of 32); any query
 * count and any num_q_heads / num_kv_heads.  bf16 at head_dim 64 or 128 runs
 * on MFMA; other element types and head dims on an fp32 VALU kernel.
 * num_splits splits each (batch, kv head)'s keys over workgroups (0 = library
 * default); the workspace must hold voom_position_free_workspace_bytes(...)
 * for the same values.  Page ids outside [0, num_pages) read page 0 and
 * table rows are read at positions clamped to [0, max_position); callers
 * validate them (voom_check_position_free_pages does, see below).
 * ------------------------------------------------------------------------- */
#define VOOM_DTYPE_BF16 0
#define VOOM_DTYPE_F16 1
#define VOOM_DTYPE_F32 2
size_t voom_position_free_workspace_bytes(int batch, int num_q_heads, int num_queries,
                                          int num_kv_heads, int head_dim, int num_keys,
                                          int dtype, int num_splits);
int voom_position_free_attention(const void* q, const void* k_pages, const void* v_pages,
                                 const int32_t* block_table, const int32_t* key_positions,
                                 const int32_t* query_positions, const void* cos_table,
                                 const void* sin_table, void* out, void* workspace,
                                 size_t ws_bytes, int batch, int num_q_heads, int num_queries,
                                 int num_kv_heads, int head_dim, int block_size, int num_pages,
                                 int num_keys, int max_position, int dtype, int table_dtype,
                                 float scale, int num_splits, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Debug bounds checks of the attention calls' index arrays.
 *
 * The attention kernels never fault on a bad index (a slot or page id out of
 * range reads slot 0; a position outside the RoPE tables is clamped), so a
 * caller's bug would give plausible numbers.  The reference raises instead:
 * IndexError/ValueError from its page pool (runtime/kv_cache.py:305-310,
 * 357-476) and ValueError from the kernel wrapper (runtime/pic_attention.py:
 * 197-213).  These calls count, into the caller-zeroed int32 status[4], what
 * the matching attention call would read out of range; the host layer raises
 * ValueError on a non-zero count.  Each is one launch; nothing traps.
 *   voom_check_block_table           for voom_paged_gqa_* and the dense MLA
 *       calls: status[0] += slot ids outside [0, num_slots) among the first
 *       ceil(ctx_lens[b] / page_tokens) columns of row b (a spilled
 *       column's -1 included); status[1] += ctx_lens outside
 *       [0, max_pages * page_tokens].
 *   voom_check_selection             for voom_mla_sparse_decode: status[0] +=
 *       slot ids outside [0, num_slots) read by a used position; status[2] +=
 *       used positions outside [0, max_pages * page_tokens); status[3] +=
 *       sel_lens outside [0, k].
 *   voom_check_position_free_pages   for voom_position_free_attention:
 *       status[0] += keys whose page id lies outside [0, num_pages);
 *       status[1] += key positions outside [0, max_position).
 * ------------------------------------------------------------------------- */
int voom_check_block_table(const int32_t* block_table, const int32_t* ctx_lens,
                           int32_t* status, int batch, int max_pages, int page_tokens,
                           int num_slots, hipStream_t stream);
int voom_check_selection(const int32_t* sel, const int32_t* sel_lens, const int32_t* block_table,
                         int32_t* status, int batch, int k, int max_pages, int page_tokens,
                         int num_slots, hipStream_t stream);
int voom_check_position_free_pages(const int32_t* block_table, const int32_t* key_positions,
                                   int32_t* status, int num_keys, int block_size, int num_pages,
                                   int max_position, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Decoder-block ops of the end-to-end decode harness (all bf16, memory-bound).
 *
 * voom_add_rms_norm: with delta, x = bf16(x + delta) in place (the residual
 * add); then out = bf16(weight * bf16(x * rsqrt(mean(x^2) + eps))), fp32
 * statistics -- mx.fast.rms_norm at runtime/layer_runner.py:263,309, with
 * Hugging Face Llama's cast order.  x, delta, out [rows, hidden], weight
 * [hidden]; hidden a multiple of 8 up to 8192; delta may be NULL.
 *
 * voom_rope_split: qkv [batch * seq, (nq + 2 nkv) * head_dim] (the fused
 * projection) -> q [batch, nq, seq, head_dim], k and v [batch, nkv, seq,
 * head_dim], q and k rotated (rotate-half RoPE, fp32 products, bf16 out) with
 * the fp32 tables cos/sin [seq, head_dim] -- mx.fast.rope at
 * runtime/layer_runner.py:99-103 plus the head split and transpose.
 *
 * voom_silu_mul: gate_up [rows, 2 * intermediate] (gate first) ->
 * out [rows, intermediate] = bf16(bf16(silu(gate)) * up) -- _silu_mul,
 * runtime/layer_runner.py:43-46,188.
 * ------------------------------------------------------------------------- */
int voom_add_rms_norm(void* x, const void* delta, const void* weight, void* out, int rows,
                      int hidden, float eps, hipStream_t stream);
int voom_rope_split(const void* qkv, const float* cos_table, const float* sin_table, void* q,
                    void* k, void* v, int batch, int seq, int num_q_heads, int num_kv_heads,
                    int head_dim, hipStream_t stream);
int voom_silu_mul(const void* gate_up, void* out, int rows, int intermediate,
                  hipStream_t stream);

/* voom_gemv_bf16: one-token projection y [n] = bf16(weight [n, k] . x [k]),
 * fp32 sums -- the _linear calls of a decode step (runtime/layer_runner.py:73,
 * 182, 186-190) at one row of activations.  With swiglu != 0, weight is the
 * fused [gate; up] projection [2n, k] and y [n] = bf16(bf16(silu(g)) * u) of
 * the bf16-rounded projections g (row r) and u (row n + r): the gate/up
 * projections and _silu_mul (layer_runner.py:186-188) in one launch.
 * k a multiple of 8 up to 2048; weight and x 16-byte aligned. */
int voom_gemv_bf16(const void* weight, const void* x, void* y, int n, int k, int swiglu,
                   hipStream_t stream);

/* voom_add_rms_norm_gemv: voom_add_rms_norm of one row followed by
 * voom_gemv_bf16 on its output, in one launch: the projection's input is
 * bf16(ln_weight * bf16(v * rsqrt(mean(v^2) + eps))) with v = bf16(x + delta)
 * (v = x when delta is NULL), and v is stored to x_out when x_out is not NULL
 * (x_out must not alias x or delta: the residual stream ping-pongs between two
 * buffers instead of being updated in place).  Bit-identical to the two ops in
 * sequence: every row statistic is summed in the same fixed order.  With
 * ln_weight NULL (and delta, x_out NULL) it is voom_gemv_bf16.  The residual
 * add and pre-norm of the dense block feeding its projections,
 * runtime/layer_runner.py:338-344. */
int voom_add_rms_norm_gemv(const void* x, const void* delta, const void* ln_weight, float eps,
                           void* x_out, const void* weight, void* y, int n, int k, int swiglu,
                           hipStream_t stream);

/* voom_lm_head_argmax: greedy next token of one row -- the index of the
 * largest bf16 logit of weight [n, k] . h (the lowest index among equal
 * logits; -0 equals +0, NaN is largest, as torch.argmax), written to
 * token[0] and, when not NULL, token_copy[0] (int64).  h is x itself, or,
 * with ln_weight, the residual-add + RMSNorm of voom_add_rms_norm_gemv (the
 * final norm).  The logits are not stored.  workspace holds one 8-byte key
 * per 16 vocabulary rows.  The final norm, lm_head and greedy sample of the
 * decode loop, runtime/engine.py:8471-8479 (argmax at :6446). */
int voom_lm_head_argmax(const void* x, const void* delta, const void* ln_weight, float eps,
                        const void* weight, int n, int k, void* workspace, size_t ws_bytes,
                        int64_t* token, int64_t* token_copy, hipStream_t stream);

/* voom_qkv_rope_append: one decode token of one sequence through the fused
 * qkv projection, RoPE and the page write -- voom_gemv_bf16 with w_qkv
 * [(nq + 2 nkv) * head_dim, k], voom_rope_split with the fp32 rows cos_row /
 * sin_row [head_dim] of the token's position, and voom_append_kv at
 * *position (a device int) through table_row [max_pages], in one launch and
 * bit-identical to the three in sequence (runtime/layer_runner.py:73-103 and
 * the cache update at :158).  q [num_q_heads, head_dim] out; k and v into the
 * pools (layouts of voom_append_kv).  head_dim a multiple of 4.  delta,
 * ln_weight, eps and x_out are the optional residual-add + RMSNorm prologue of
 * voom_add_rms_norm_gemv (ln_weight NULL: x is the projection input).  With
 * rope_rows > 0, cos_row / sin_row are tables [rope_rows, head_dim] and the
 * row of *position is used (clamped into the table), so a captured step needs
 * no per-token table work. */
int voom_qkv_rope_append(const void* w_qkv, const void* x, const void* delta,
                         const void* ln_weight, float eps, void* x_out, const float* cos_row,
                         const float* sin_row, void* q, void* k_pool, void* v_pool,
                         const int32_t* table_row, const int32_t* position, int num_q_heads,
                         int num_kv_heads, int head_dim, int k, int page_tokens, int max_pages,
                         int num_slots, int rope_rows, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Page writes and reads.
 *
 * voom_append_kv writes L new tokens per sequence into the pools at logical
 * positions pos[b] .. pos[b]+L-1 through the block table (slot write, no
 * concatenation).  Replaces the tail concatenation and page close of
 * PagedKVCache.update (runtime/kv_paged.py:143-158).
 *   k_new, v_new [batch, num_kv_heads, L, head_dim] bf16 (contiguous)
 *   positions    [batch] int32 first logical position of the new tokens
 *
 * voom_gather_kv materialises the logical K/V [batch, num_kv_heads, S, head_dim]
 * (positions 0..S-1) from the pools: the reference's concatenated return value
 * of PagedKVCache.update (runtime/kv_paged.py:176-181).
 * ------------------------------------------------------------------------- */
int voom_append_kv(const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                   const int32_t* block_table, const int32_t* positions, int batch,
                   int num_kv_heads, int new_tokens, int head_dim, int page_tokens,
                   int max_pages, int num_slots, hipStream_t stream);
int voom_gather_kv(const void* k_pool, const void* v_pool, const int32_t* block_table,
                   void* k_out, void* v_out, int batch, int num_kv_heads, int seq_len,
                   int head_dim, int page_tokens, int max_pages, int num_slots,
                   hipStream_t stream);

/* Token-row pages (the paged MLA latent cache, pool [num_slots, page_tokens,
 * row_elems]): voom_append_rows writes src [batch, new_tokens, row_elems] at
 * positions[b] + t (the latent append of KVCache.update_latent,
 * runtime/kv_cache.py:99-105, as a slot write); voom_gather_rows materialises
 * [batch, seq_len, row_elems] in logical order (its concatenated return). */
int voom_append_rows(const void* src, void* pool, const int32_t* block_table,
                     const int32_t* positions, int batch, int new_tokens, int row_elems,
                     int page_tokens, int max_pages, int num_slots, hipStream_t stream);
int voom_gather_rows(const void* pool, const int32_t* block_table, void* dst, int batch,
                     int seq_len, int row_elems, int page_tokens, int max_pages, int num_slots,
                     hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Byte-plane codec (bit-exact).
 *
 * A little-endian 16-bit element e splits into lo = e & 0xff and hi = e >> 8;
 * the planes hold byte 0 resp. byte 1 of every element in element order.
 * Replaces formats/packed.py:49-50 / 277-282 (lo = raw[0::2], hi = raw[1::2])
 * and the inverse interleave of packed.py:376-378.
 *
 * The _slots variants gather (split) or scatter (merge) whole pool slots of
 * slot_bytes bytes each: slot i of the plane stream is slot slots[i] of the
 * pool.  slot_bytes must be a multiple of 64.  `slots` is a device int32
 * array of n_slots entries, each in [0, num_slots).
 * ------------------------------------------------------------------------- */
int voom_byteplane_split(const void* src, void* lo, void* hi, size_t n_elems,
                         hipStream_t stream);
int voom_byteplane_merge(const void* lo, const void* hi, void* dst, size_t n_elems,
                         hipStream_t stream);
/* sums (NULL = none): per listed slot i, sums[i] += the slot's checksum, a
 * position-keyed word hash (word j of the slot adds fmix32(word + j *
 * 0x9E3779B9) mod 2^32, fmix32 = MurmurHash3's finaliser).  The split sums the
 * slot it reads, the merge the words it writes back, so equal sums mean the
 * spilled bytes came back unchanged.  The caller zeroes sums first.  The
 * reference has no spill checksum; this is the pinned-arena and page-file
 * integrity check of this build. */
int voom_byteplane_split_slots(const void* pool, const int32_t* slots, int n_slots,
                               size_t slot_bytes, int num_slots, void* lo, void* hi,
                               uint32_t* sums, hipStream_t stream);
int voom_byteplane_merge_slots(const void* lo, const void* hi, void* pool,
                               const int32_t* slots, int n_slots, size_t slot_bytes,
                               int num_slots, uint32_t* sums, hipStream_t stream);
/* Compares n checksums: status[0] += the number of mismatches, and the first
 * mismatch stores ``tag`` (non-zero) in status[1] if it is still 0.  The
 * status words are sticky until the caller clears them. */
int voom_page_sums_verify(const uint32_t* expected, const uint32_t* got, int n, int tag,
                          int32_t* status, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Spill records: pool slots <-> one record in pinned host memory, moved by
 * the codec kernel itself (no staging buffer, no copy engine).
 *
 * Replaces the page move of the reference's spill (runtime/kv_paged.py:77-96,
 * planes as formats/packed.py:49-50) and reload (runtime/kv_paged.py:98-113).
 *
 * A record of R slots over T pool tensors (T <= 4; tensor t's slots are
 * slot_bytes[t] bytes, a multiple of 64, h_t = slot_bytes[t] / 2) is laid out
 * as the low planes of every tensor (tensor t: R * h_t bytes, record slot r at
 * r * h_t), then the high planes in the same arrangement, then, with
 * checksums, int32 [T][R] (the checksum of voom_byteplane_split_slots).
 * Listed slot i (pool slot slots[i] of every tensor) is record slot first + i;
 * first + n_slots <= rec_slots.  `slots` is an int32 array of n_slots
 * entries in device or pinned host memory (read by the kernel, so a host list
 * needs no upload; it must stay unchanged until the call has run); entries
 * outside [0, num_slots[t]) are skipped.
 *
 * `record` is pinned host memory (hipHostMalloc) or device memory; the call
 * looks the record and the slot list up and refuses pageable or too-short
 * memory.  Host
 * records are written and read with system-scope accesses, so the host sees
 * a spilled record once the stream has passed the call, and a reload reads
 * what the host last wrote.  Both calls run on `stream`, which must be
 * ordered after the writes of the slots they read.
 * ------------------------------------------------------------------------- */
/* Sets the record kernels up on the current device, so that the first spill
 * does not pay their one-time launch setup (optional; idempotent). */
int voom_record_prepare(void);
/* Splits listed slots into the record; with_sums stores their checksums. */
int voom_spill_record(const void* const* pools, const size_t* slot_bytes, const int* num_slots,
                      int n_tensors, const int32_t* slots, int n_slots, void* record,
                      int rec_slots, int first, int with_sums, hipStream_t stream);
/* Merges record slots back into listed pool slots.  tag != 0: the checksum
 * of every merged slot is compared with the record's; each mismatch adds 1
 * to status[0] and the first stores tag in status[1] if it is still 0
 * (device int32[2], as voom_page_sums_verify). */
int voom_reload_record(const void* record, int rec_slots, int first, void* const* pools,
                       const size_t* slot_bytes, const int* num_slots, int n_tensors,
                       const int32_t* slots, int n_slots, int tag, int32_t* status,
                       hipStream_t stream);
/* Copies `rows` rows of `width` bytes, row r from src + r * src_pitch to
 * dst + r * dst_pitch, as one asynchronous transfer on `stream` (the copy
 * engine; either side pinned host or device memory; width <= both pitches).
 * The staged reload of the reference's page load (runtime/kv_paged.py:98-113)
 * uses it to move one byte plane of many spilled pages, each in its own host
 * record at a constant spacing, in one transfer instead of one per page. */
int voom_copy_rows(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width,
                   size_t rows, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VOOM_HIP_H */
