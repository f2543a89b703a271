/*
 * qattn.h -- C ABI of the MI355X (gfx950) ancestor-sparse tree-verify
 * attention library, libqattn.so.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * launches asynchronously on the given HIP stream (hipStream_t passed as
 * void*, NULL = the legacy default stream) and is HIP-graph capturable.
 * Outputs and workspaces belong to the caller.  No entry point allocates
 * memory, synchronises or zeroes anything behind the caller's back.
 *
 * The subtree kernel's work-schedule counters live in a static device array
 * (2 MiB per device, part of the library's code object).  qattn_init() sets
 * it up on the current device; until then every launch on that device runs
 * the static schedule (same results, slower).  Each launch leaves its
 * counters at zero.  A counter slot only serves launches that cannot overlap:
 *   - an uncaptured launch uses the slot of its stream (launches on one
 *     stream run in order); 64 streams per device get a slot, launches on
 *     further streams run the static schedule;
 *   - the launches recorded into a graph by one capture sequence on one
 *     stream share a slot for every replay (they run in order, and replays
 *     of one graph executable run in order); 192 such slots per device are
 *     held at a time, each until its graph and the executables made from it
 *     are destroyed; beyond that, recorded launches use the static schedule.
 *     As with any memory a capture records, two graph executables
 *     instantiated from one capture must not run at the same time.
 * qattn_sched_info() reports the slots in use and the launches that ran each
 * schedule.  Calls are thread-safe (the slot table is guarded by a mutex).
 * Return value: QATTN_OK (0) or a negative QATTN_ERR_* code; the message of
 * the last failure on the calling thread is qattn_last_error().
 *
 * Conventions shared by the entry points
 *   - Tensors are [tokens, heads, head_dim] with strides given as
 *     {stride_token, stride_head, stride_dim} in ELEMENTS; stride_dim must be
 *     1 and every row must start on a 16-byte boundary (else
 *     QATTN_ERR_LAYOUT; callers copy to a contiguous layout).
 *   - dtype is QATTN_DTYPE_F16 or QATTN_DTYPE_BF16 for q, k, v and o alike;
 *     arithmetic is fp32; o is rounded once (nearest even).
 *   - head_dim is 32, 64 or 128.  num_q_heads must be a multiple of
 *     num_kv_heads (GQA: q head h reads kv head h / (num_q_heads/num_kv_heads),
 *     the mapping of repeat_kv; num_kv_heads == num_q_heads is the reference
 *     layout).
 *   - cu_seqlens is a DEVICE int32 array [batch + 1] of sequence offsets;
 *     max_seqlen bounds every sequence length (tokens at or beyond it are not
 *     computed).  A sequence whose offsets are decreasing, negative or beyond
 *     total_tokens is skipped (its output rows are left untouched).
 *   - scale multiplies q.k (the reference fixes it to 1/sqrt(head_dim)); the
 *     tree-only entry points take any finite scale, the prefix entry points
 *     require scale > 0.
 *   - lse (optional, may be NULL) is fp32 [tokens, num_q_heads] with strides
 *     {stride_token, stride_head}: lse = m + ln(sum exp(s - m)).
 */
#ifndef QATTN_H_
#define QATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QATTN_OK 0
#define QATTN_ERR_ARG (-1)       /* null pointer, bad size or inconsistent shape */
#define QATTN_ERR_DTYPE (-2)     /* dtype not fp16/bf16 */
#define QATTN_ERR_HEAD_DIM (-3)  /* head_dim not in {32, 64, 128} */
#define QATTN_ERR_LAYOUT (-4)    /* stride_dim != 1 or a row not 16-byte aligned */
#define QATTN_ERR_WORKSPACE (-5) /* workspace missing or too small */
#define QATTN_ERR_HIP (-6)       /* HIP launch/runtime error */

#define QATTN_DTYPE_F16 0
#define QATTN_DTYPE_BF16 1

/* Kernel selection for qattn_tree_fwd (QATTN_ALGO_AUTO picks per shape). */
#define QATTN_ALGO_AUTO 0
#define QATTN_ALGO_GATHER 1  /* one row group per (token, head), gathers from global */
#define QATTN_ALGO_SUBTREE 2 /* subtree tiles staged in LDS (heap trees only) */

/* Library version string. */
const char *qattn_version(void);

/*
 * Set up the library on the CURRENT device (no reference counterpart: the
 * Triton module has no device state).  Looks up the device address of the
 * schedule-counter array and zeroes it, synchronously, on a private stream.
 * Call it once per device before the first attention call there, outside
 * graph capture; later calls return at once.  Without it every call still
 * works, with the subtree kernel on its static schedule.
 */
int qattn_init(void);

/*
 * Schedule-counter use on the CURRENT device (no reference counterpart: it
 * makes the subtree kernel's schedule choice visible to tests and benchmarks).
 * info[0] streams holding an eager slot, info[1] graph-capture slots held,
 * info[2] subtree launches (eager or recorded) given counters, info[3]
 * launches that wanted counters and ran the static schedule because no slot
 * was free (launches before qattn_init are not counted), info[4] and info[5]
 * the eager and captured slot capacities.
 */
int qattn_sched_info(int64_t info[6]);

/* Message of the last failed call on this thread ("" if none). */
const char *qattn_last_error(void);

/*
 * Ancestor-sparse attention over complete b-ary heap-indexed trees.
 *
 * Replaces _ragged_attn_sparse_kernel / _ragged_attn_sparse_kernel_lse /
 * _ragged_attn_sibling_kernel(_lse) (src/ragged_attn.py:262-497, 1206-1420)
 * as launched by ragged_attention (:1080-1166), ragged_attention_with_lse
 * (:499-572) and the sibling wrappers (:1423-1556).
 *
 * For token t of sequence s (local index x = t - cu[s]) and q head h:
 *   A(x) = { c_i : c_0 = x, c_{i+1} = max(c_i - 1, 0) / b, c_i != c_{i-1},
 *            i = 0..max_depth }
 *   o[t,h] = softmax_{a in A(x)}(scale q[t,h].k[cu[s]+a,kvh]) . v[cu[s]+a,kvh]
 */
int qattn_tree_fwd(const void *q, const int64_t q_stride[3],
                   const void *k, const int64_t k_stride[3],
                   const void *v, const int64_t v_stride[3],
                   void *o, const int64_t o_stride[3],
                   float *lse, const int64_t lse_stride[2],
                   const int32_t *cu_seqlens, int32_t batch, int32_t max_seqlen,
                   int64_t total_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                   int32_t head_dim, int32_t branching_factor, int32_t max_depth,
                   float scale, int32_t dtype, int32_t algo, void *stream);

/*
 * Ancestor-sparse attention with an explicit parent array (irregular trees).
 *
 * Replaces _ragged_attn_parents_kernel_lse (src/ragged_attn.py:588-714)
 * launched by ragged_attention_with_parents (:716-795).  parents is a DEVICE
 * int32 array [total_tokens] of sequence-local parent indices; a root must
 * self-loop (parents[root] == root).  The walk is c_{i+1} = parents[cu[s]+c_i],
 * attending c_i iff c_i != c_{i-1}, for i = 0..max_depth.  A parent outside
 * [0, sequence length) ends the walk (the reference leaves it undefined).
 */
int qattn_tree_parents_fwd(const void *q, const int64_t q_stride[3],
                           const void *k, const int64_t k_stride[3],
                           const void *v, const int64_t v_stride[3],
                           void *o, const int64_t o_stride[3],
                           float *lse, const int64_t lse_stride[2],
                           const int32_t *cu_seqlens, const int32_t *parents,
                           int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t max_depth, float scale, int32_t dtype, void *stream);

/*
 * Ancestor-sparse attention reading K/V from a paged cache.
 *
 * Replaces _ragged_attn_paged_kernel (src/ragged_attn.py:822-929) launched by
 * ragged_attention_paged (:932-1003).  k_cache / v_cache are
 * [num_pages, page_size, num_kv_heads, head_dim] with strides
 * {page, slot, head, dim}; page_table is a DEVICE int32 [batch, pt_cols]
 * array (row stride pt_cols).  Ancestor position c of sequence s lives at
 * page page_table[s, c / page_size], slot c % page_size.  A page index outside
 * [0, num_pages) or a logical page beyond pt_cols skips that ancestor; a query
 * that attends nothing gets o = 0 and lse = -inf.  algo selects the kernel as
 * for qattn_tree_fwd: the subtree kernel stages each tile's rows once through
 * LDS and takes batch * pt_cols <= 2048 page-table entries.
 */
int qattn_tree_paged_fwd(const void *q, const int64_t q_stride[3],
                         const void *k_cache, const int64_t k_stride[4],
                         const void *v_cache, const int64_t v_stride[4],
                         void *o, const int64_t o_stride[3],
                         float *lse, const int64_t lse_stride[2],
                         const int32_t *cu_seqlens, const int32_t *page_table,
                         int32_t pt_cols, int32_t num_pages, int32_t page_size,
                         int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                         int32_t branching_factor, int32_t max_depth, float scale,
                         int32_t dtype, int32_t algo, void *stream);

/*
 * Ancestor index table of the heap walk (parents == NULL) or the
 * explicit-parent walk, computed by the same device code as the attention
 * kernels.  out is a DEVICE int32 [total_tokens, max_depth + 1] array:
 * out[t, i] = c_i if step i attends, else -1.  No reference counterpart as an
 * entry point: it exposes the walk of src/ragged_attn.py:323-377 / :650-698
 * so index sets can be checked bit-exactly.
 */
int qattn_ancestors(const int32_t *cu_seqlens, const int32_t *parents, int32_t batch,
                    int32_t max_seqlen, int64_t total_tokens, int32_t branching_factor,
                    int32_t max_depth, int32_t *out, void *stream);

/*
 * Walk export, a test hook (no reference counterpart; it exposes the walk of
 * src/ragged_attn.py:323-377 / :650-698 as each kernel executes it).  While
 * out is non-null, the attention calls made on the calling thread run their
 * kernels' walk-export instantiations: the same outputs, plus, for every
 * query (packed token t, q head h) they compute, the ancestor set the
 * kernel used, out[(t * num_q_heads + h) * (max_depth + 1) + i] = the node
 * attended at walk step i, or -1.  Subtree kernel: the query's row mask
 * decoded through the row map its K/V loads were issued with; gather walk:
 * the node each step loads; fused prefix epilogue: the node of the staged
 * LDS row each step reads.  -2 at step 0 marks an inconsistency (a mask bit
 * on a row without a node, two rows at one step, a Q row staged from another
 * query).  Entries of queries no kernel computes are left as they were.
 * Calls over packed cu_seqlens, fp16 or bf16, with or without lse (the
 * uniform-batch qattn_ragged_tree_attn_fwd returns QATTN_ERR_ARG);
 * out is a DEVICE int32 array of total_tokens * num_q_heads * (max_depth+1)
 * entries.  NULL turns it off.
 */
int qattn_debug_walk(int32_t *out);

/*
 * Tree-verify attention with a prefix KV cache that every tree query attends
 * in full, plus its own ancestors among the tree tokens.
 *
 * Replaces _ragged_attn_hybrid_kernel (src/ragged_attn.py:1709-1848) launched
 * by ragged_attention_hybrid (:1851-1888), and the three-step caller pipeline
 * "prefix flash attention + ragged_attention_with_lse + fused_lse_merge"
 * (scripts/benchmark_micro.py:568-593, scripts/e2e_benchmark.py:1394-1502).
 *
 * Prefix key/value row j of sequence s, kv head g, is
 *   k_prefix + s*kp_stride[0] + j*kp_stride[1] + g*kp_stride[2]
 * (kp_stride[0] == 0 shares one prefix across the batch; K/V heads are GQA
 * heads, never repeated).  Prefix strides are multiples of 8 elements with
 * 16-byte aligned pointers, and the token strides kp_stride[1], vp_stride[1]
 * are non-negative and below 2^25 elements (else QATTN_ERR_LAYOUT): the
 * kernel addresses a 64-key block with 32-bit byte offsets.  Tree key/value row of local ancestor x of sequence
 * s is  tree_seq_stride ? s*tree_seq_stride + tree_row0 + x : cu_seqlens[s] + x
 * (the reference hybrid layout [B*(L+N), H, D] is tree_seq_stride = L+N,
 * tree_row0 = L).  The prefix is computed with v_mfma_f32_32x32x16 products
 * (16x16x32 for half-height split tiles) in splits along the prefix; the
 * split states are merged into the ancestor walk, which normalises once.  workspace (device, 256-byte aligned, at least
 * qattn_prefix_workspace_bytes() bytes for the same sizes and num_splits)
 * holds the split states; num_splits 0 picks a split count for 256 CUs.
 * prefix_len 0 reduces to qattn_tree_fwd (workspace unused).
 */
int64_t qattn_prefix_workspace_bytes(int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t prefix_len, int32_t num_splits);

int qattn_prefix_tree_fwd(const void *q, const int64_t q_stride[3],
                          const void *k, const int64_t k_stride[3],
                          const void *v, const int64_t v_stride[3],
                          const void *k_prefix, const int64_t kp_stride[3],
                          const void *v_prefix, const int64_t vp_stride[3],
                          int32_t prefix_len,
                          void *o, const int64_t o_stride[3],
                          float *lse, const int64_t lse_stride[2],
                          const int32_t *cu_seqlens, int32_t batch, int32_t max_seqlen,
                          int64_t total_tokens, int64_t tree_seq_stride, int64_t tree_row0,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t branching_factor, int32_t max_depth, float scale,
                          int32_t dtype, void *workspace, int64_t workspace_size,
                          int32_t num_splits, void *stream);

/*
 * Attention of query tokens over a prefix KV cache only (no tree keys), with
 * LSE: the prefix pass of the reference's verify pipelines, in the layout of
 * qattn_prefix_tree_fwd, GQA-native.
 *
 * Replaces flashinfer.single_prefill_with_kv_cache_return_lse as the
 * reference benchmark calls it (scripts/benchmark_micro.py:574-580, a prefix
 * [L, H, D] shared by every query: kp_stride[0] == 0) and the aten flash
 * prefix pass with LSE of the E2E verify step (scripts/e2e_benchmark.py:
 * 1438-1448, one prefix per sequence).  Query token t of sequence s (rows
 * cu_seqlens[s] .. cu_seqlens[s+1]-1) attends all prefix_len >= 1 rows of
 * sequence s's prefix.  Workspace sized by qattn_prefix_workspace_bytes()
 * with the same arguments; the split count and prefix kernel are those of
 * qattn_prefix_tree_fwd, so the two calls time the prefix alone and the
 * prefix plus tree.
 */
int qattn_prefix_fwd(const void *q, const int64_t q_stride[3],
                     const void *k_prefix, const int64_t kp_stride[3],
                     const void *v_prefix, const int64_t vp_stride[3], int32_t prefix_len,
                     void *o, const int64_t o_stride[3], float *lse, const int64_t lse_stride[2],
                     const int32_t *cu_seqlens, int32_t batch, int32_t max_seqlen,
                     int64_t total_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, float scale, int32_t dtype, void *workspace,
                     int64_t workspace_size, int32_t num_splits, void *stream);

/*
 * The same over an explicit parent array (EAGLE-3 dynamic trees) instead of a
 * heap tree: parents as in qattn_tree_parents_fwd, everything else as in
 * qattn_prefix_tree_fwd (same workspace size).
 *
 * Replaces the reference E2E verify composition for a tree with parents:
 * prefix flash attention with LSE + ragged_attention_with_parents +
 * fused_lse_merge (scripts/e2e_benchmark.py:1427-1496, the tree_parents
 * branch at :1466-1474; kernels src/ragged_attn.py:588-714, 1575-1616), in
 * one call, GQA-native, without the intermediate O/LSE tensors.
 */
int qattn_prefix_tree_parents_fwd(const void *q, const int64_t q_stride[3],
                                  const void *k, const int64_t k_stride[3],
                                  const void *v, const int64_t v_stride[3],
                                  const void *k_prefix, const int64_t kp_stride[3],
                                  const void *v_prefix, const int64_t vp_stride[3],
                                  int32_t prefix_len,
                                  void *o, const int64_t o_stride[3],
                                  float *lse, const int64_t lse_stride[2],
                                  const int32_t *cu_seqlens, const int32_t *parents,
                                  int32_t batch, int32_t max_seqlen, int64_t total_tokens,
                                  int64_t tree_seq_stride, int64_t tree_row0,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t max_depth, float scale, int32_t dtype,
                                  void *workspace, int64_t workspace_size,
                                  int32_t num_splits, void *stream);

/*
 * Tree verification over [B, H, N, D] views, as the model's attention layer
 * holds them: no cu_seqlens, no packing, no copies.
 *
 * Replaces _ragged_tree_attn (scripts/e2e_benchmark.py:1394-1502): the
 * prefix split and .contiguous() copies (:1430-1431), flash prefix attention
 * with LSE (:1438-1448), the permute/contiguous repacks of Q and the tree K/V
 * (:1455-1462), the cu arange (:1464), the tree kernel over a heap tree or
 * over tree_parents (:1470-1478), the output permutes (:1482-1487) and
 * fused_lse_merge (:1496) -- in one call, GQA-native.
 *   q, o   [batch, num_q_heads, num_tree, head_dim], 4 element strides each
 *          (torch order: batch, head, token, dim; stride_dim 1, rows and the
 *          batch stride 16-byte aligned);
 *   k, v   [batch, num_kv_heads, num_prefix + num_tree, head_dim], 4 strides:
 *          rows 0 .. num_prefix-1 of each sequence are its prefix (all
 *          visible to every tree token), the remaining num_tree rows its tree
 *          tokens in BFS order.  For batch > 1 the batch stride of k and of v
 *          must be the same positive multiple of its token stride (true of
 *          any dense layout with the token dimension inside the batch one);
 *   lse    null, or fp32 [batch, num_q_heads, num_tree] with 3 strides:
 *          log-sum-exp over prefix and ancestors (natural log);
 *   parents null: heap tree of branching_factor; else sequence-local parent
 *          per tree token (the root its own parent, or negative) of sequence
 *          s at parents[s * parents_stride + i] -- parents_stride 0 shares
 *          one [num_tree] array (the reference's tree_parents) between all
 *          sequences, num_tree gives one array per sequence.
 * Query head h reads kv head h / (num_q_heads / num_kv_heads).  workspace as
 * in qattn_prefix_tree_fwd, sized by qattn_prefix_workspace_bytes(batch,
 * num_tree, batch * num_tree, num_q_heads, num_kv_heads, head_dim,
 * num_prefix, num_splits); num_prefix 0 needs none.
 */
int qattn_ragged_tree_attn_fwd(const void *q, const int64_t q_stride[4],
                               const void *k, const int64_t k_stride[4],
                               const void *v, const int64_t v_stride[4],
                               void *o, const int64_t o_stride[4],
                               float *lse, const int64_t lse_stride[3],
                               const int32_t *parents, int64_t parents_stride,
                               int32_t batch, int32_t num_tree, int32_t num_prefix,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t branching_factor, int32_t max_depth, float scale,
                               int32_t dtype, void *workspace, int64_t workspace_size,
                               int32_t num_splits, void *stream);

/*
 * qattn_ragged_tree_attn_fwd without the workspace arguments, for callers
 * that cannot allocate (code under HIP graph capture that must not touch an
 * allocator, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference: it keeps the prefix split states in the
 * library's static device array `scratch` (32 MiB per device, held until the
 * process ends) and calls no allocating routine.  The split count is chosen
 * as by qattn_ragged_tree_attn_fwd; with num_splits 0 it is lowered until
 * the split states fit the 32 MiB (one split needs none), an explicit
 * num_splits whose states do not fit returns QATTN_ERR_WORKSPACE.  Every
 * call on a device shares that device's scratch: calls that overlap in time
 * on one device (other streams, other threads) race and must not be issued.
 * Everything else, including the results, is as qattn_ragged_tree_attn_fwd.
 */
int qattn_ragged_tree_attn_fwd_noalloc(const void *q, const int64_t q_stride[4],
                                       const void *k, const int64_t k_stride[4],
                                       const void *v, const int64_t v_stride[4],
                                       void *o, const int64_t o_stride[4],
                                       float *lse, const int64_t lse_stride[3],
                                       const int32_t *parents, int64_t parents_stride,
                                       int32_t batch, int32_t num_tree, int32_t num_prefix,
                                       int32_t num_q_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t branching_factor,
                                       int32_t max_depth, float scale, int32_t dtype,
                                       int32_t num_splits, void *stream);

/*
 * Two-state softmax merge.
 *
 * Replaces _fused_lse_merge_kernel (src/ragged_attn.py:1575-1616) launched by
 * fused_lse_merge (:1619-1653):
 *   w_p = exp(lse_p - max), w_t = exp(lse_t - max),
 *   out = (w_p o_p + w_t o_t) / max(w_p + w_t, 1e-8).
 * o_pre, o_tree, out are [B, H, Nq, D] with 4 element strides each (any
 * layout with stride_dim 1 and 16-byte aligned rows); lse_pre, lse_tree are
 * fp32 [B, H, Nq] with 3 strides each.
 */
int qattn_lse_merge(const float *lse_pre, const int64_t lse_pre_stride[3],
                    const float *lse_tree, const int64_t lse_tree_stride[3],
                    const void *o_pre, const int64_t o_pre_stride[4],
                    const void *o_tree, const int64_t o_tree_stride[4],
                    void *out, const int64_t out_stride[4],
                    int32_t B, int32_t H, int32_t Nq, int32_t head_dim,
                    int32_t dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QATTN_H_ */
