/*
 * spruce_hip.h — C ABI of libspruce_hip.so, the MI355X (gfx950) kernels behind
 * SPRUCE's sparse-prefill hot path.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; the caller owns every buffer (inputs,
 *     outputs and workspace).  Nothing here allocates device memory.
 *   - Strides are in ELEMENTS (not bytes), int64, in the logical order named
 *     next to each argument.  The innermost (head_dim) stride must be 1.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Launches
 *     are asynchronous; no entry point synchronises the host.
 *   - Return value: 0 on success, SPRUCE_EINVAL (-1) for an invalid argument,
 *     or a positive hipError_t from the launch.  spruce_last_error() copies the
 *     message of the most recent failure on the calling thread.
 *   - Functions hold no global mutable state besides that thread-local error
 *     slot, so they are reentrant.
 *
 * Each declaration cites the reference (Rand0miz/spruce-research) interface
 * it replaces as file:line.
 */
#ifndef SPRUCE_HIP_H
#define SPRUCE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPRUCE_OK 0
#define SPRUCE_EINVAL (-1)

/* Element type of Q/K/V and of the attention output (U8: boolean attention
 * masks only, nonzero = attend). */
#define SPRUCE_DTYPE_BF16 0
#define SPRUCE_DTYPE_F16 1
#define SPRUCE_DTYPE_F32 2
#define SPRUCE_DTYPE_U8 3

/* Layouts of a projected key-prototype table of N nodes with Pk prototypes of
 * P floats each: ROWS [N, Pk, P] (one prototype per row); INTERLEAVED
 * [N, P/4, Pk, 4] (a node's prototypes interleaved by 4-float group, so the
 * Pk prototypes' floats e..e+3 of one node are one contiguous 16*Pk bytes). */
#define SPRUCE_KP_ROWS 0
#define SPRUCE_KP_INTERLEAVED 1

/* Kernel variants, in the order of the reference's KERNEL_VARIANTS tuple
 * (kernels/seerattention_direct_index_triton.py:17-23).  All variants compute
 * the same attention; they differ only in launch shape (and, for PRESCALE, in
 * rounding Q*scale*log2(e) to the MFMA input type, as the reference ablation
 * does at kernels/seerattention_direct_index_triton.py:61-63). */
#define SPRUCE_VARIANT_SINGLE_HEAD 0
#define SPRUCE_VARIANT_SINGLE_HEAD_CAUSAL 1
#define SPRUCE_VARIANT_SINGLE_HEAD_PRESCALE 2
#define SPRUCE_VARIANT_SINGLE_HEAD_QTILE 3
#define SPRUCE_VARIANT_TILED_GQA 4

/* Copies the last error message of the calling thread into buf (always
 * NUL-terminated when n > 0).  Returns the message length. */
int spruce_last_error(char* buf, size_t n);

/* Library version string, e.g. "spruce_hip 0.1 gfx950". */
const char* spruce_version(void);

/*
 * Block-sparse causal GQA prefill over a padded direct-index list.
 * Replaces direct_index_sparse_triton
 * (kernels/seerattention_direct_index_triton.py:339-416).
 *
 *   q   [B, Hq,  T, D]  strides qs   (logical order b, head, token, dim)
 *   k,v [B, Hkv, T, D]  strides ks, vs
 *   idx [B, Hkv, ceil(T/64), K] int32, strides is; entries < 0 are skipped,
 *       entries above the query block are ignored (their keys are all in the
 *       future), duplicates are attended twice exactly as listed.
 *   out [B, Hq, T, D]   strides os (the reference passes the permuted strides
 *       of a contiguous [B, T, Hq, D] buffer).
 *   D in {64, 128}; Hq % Hkv == 0; block size fixed at 64 tokens.
 * A query block whose list holds no usable block writes zeros.
 */
int spruce_sparse_prefill_index(
    const void* q, const int64_t qs[4],
    const void* k, const int64_t ks[4],
    const void* v, const int64_t vs[4],
    const int32_t* idx, const int64_t is[4], int64_t K,
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
    float scale, int dtype, int variant,
    void* out, const int64_t os[4],
    void* stream);

/*
 * Dense causal GQA prefill: every key block 0..qb of every query block, in
 * order (the all-causal-blocks case of the entry points above), with the
 * same q/k/v/out layouts and limits.  Replaces the fused causal SDPA call of
 * the reference's capture hooks (teacher/chunked_extract.py:155-161,
 * :175-181); out written through its strides, e.g. [B, T, Hq, D] as the hooks
 * return it.
 * With q_grouped and k_protos non-NULL the same pass also emits the
 * selector features of those hooks (:145-148, :170-173) from the tiles it
 * holds:
 *   q_grouped [B, Hkv, T, D] contiguous: _group_avg_tokens (:75-80) of q;
 *   k_protos  [B, Hkv, ceil(T/64), P, D] contiguous: _proto_pool_seq(k, 64,
 *             P) (:27-72);
 * bit for bit equal to spruce_group_avg_tokens / spruce_proto_pool.  Capture
 * needs dtype bf16 or f16, Hq/Hkv <= 8, 1 <= P <= 65 and 16-byte aligned
 * q_grouped / k_protos; pooling q_grouped with spruce_proto_pool (G == H)
 * gives the query prototypes.
 */
int spruce_causal_prefill(
    const void* q, const int64_t qs[4],
    const void* k, const int64_t ks[4],
    const void* v, const int64_t vs[4],
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
    float scale, int dtype,
    void* out, const int64_t os[4],
    void* q_grouped, void* k_protos, int64_t P,
    void* stream);

/*
 * Same computation over a CSR list (variable row lengths).  Rows are the
 * (b, kv_head, query_block) triples in row-major order; row r lists
 * indices[indptr[r] .. indptr[r+1]).  indptr has B*Hkv*ceil(T/64)+1 int32
 * entries and indices has nnz entries; row bounds are clamped to [0, nnz].
 * row_order (optional, may be NULL) holds a permutation of the rows that sets
 * the dispatch order (heaviest first balances the variable lengths); entries
 * outside [0, rows) are skipped.
 * No reference counterpart: the reference carries only the padded layout;
 * this is the variable-density form of spruce_sparse_prefill_index.
 */
int spruce_sparse_prefill_csr(
    const void* q, const int64_t qs[4],
    const void* k, const int64_t ks[4],
    const void* v, const int64_t vs[4],
    const int32_t* indptr, const int32_t* indices, int64_t nnz, const int32_t* row_order,
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
    float scale, int dtype, int variant,
    void* out, const int64_t os[4],
    void* stream);

/*
 * Same computation over a boolean block mask.
 * Replaces block_sparse_triton (kernels/seerattention_triton.py:71-90), and
 * additionally accepts native-GQA K/V (Hkv < Hq).
 *   mask [B, Hm, Qb, >=Qb] uint8 (torch.bool), strides ms, with Hm == Hq
 *        (per query head, the reference layout of
 *        kernels/sparse_prefill.py:16-39) or Hm == Hkv (per KV head).
 *   Only columns 0..query_block of each row are read, as the reference
 *   kernel scans them (kernels/seerattention_triton.py:60-65).
 */
int spruce_sparse_prefill_mask(
    const void* q, const int64_t qs[4],
    const void* k, const int64_t ks[4],
    const void* v, const int64_t vs[4],
    const uint8_t* mask, const int64_t ms[4], int64_t Hm,
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
    float scale, int dtype, int variant,
    void* out, const int64_t os[4],
    void* stream);

/*
 * The padded direct-index computation plus residual summaries.  Replaces the
 * residual_summaries=True branch of sparse_prefill_attention_forward
 * (sparse/attention.py:163-182, 226-265): each row's softmax also covers one
 * extra key per (listed tree node, prototype) -- the node's summary key and
 * value, with log(count) added to its score and no causal mask; prototypes
 * with count 0 (log count -inf) and nodes < 0 or >= N add nothing.
 *   nodes        [B, Hkv, Qb, S] int32, strides ns (a layer slice of the
 *                residual_summary_nodes tensor, trailing -1 padding).
 *   sum_keys, sum_values  [B, Hkv, N, P, D] contiguous (16-byte aligned),
 *                sum_log_counts float32 [B, N, P] contiguous: the
 *                KVSummaryTable spruce_kv_summary writes, N tree nodes.
 *   sum_dtype    element type of sum_keys / sum_values: SPRUCE_DTYPE_F32
 *                (the table as written), or the 16-bit input dtype (a copy
 *                rounded to nearest even, which the kernel stages like a key
 *                block: same results, half the bytes and no conversion).
 * The summary keys and values are rounded to the MFMA input type (bf16, or
 * f16 for f16 inputs) like the key blocks.
 */
int spruce_sparse_prefill_index_summaries(
    const void* q, const int64_t qs[4],
    const void* k, const int64_t ks[4],
    const void* v, const int64_t vs[4],
    const int32_t* idx, const int64_t is[4], int64_t K,
    const int32_t* nodes, const int64_t ns[4], int64_t S,
    const void* sum_keys, const void* sum_values, const float* sum_log_counts, int sum_dtype,
    int64_t N, int64_t P,
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
    float scale, int dtype, int variant,
    void* out, const int64_t os[4],
    void* stream);

/*
 * spruce_sparse_prefill_index (or _summaries when S > 0) for padded batches:
 * the padded-batch prefill of sparse_prefill_attention_forward
 * (sparse/attention.py:147-150 reduce the 4-D decoder mask to key validity,
 * :225-229 add it to the scores).  key_valid uint8 [B, T] (batch stride kvs
 * elements, tokens contiguous): nonzero marks a real token; a key with
 * key_valid == 0 gets no weight in any row.  Pass nodes = NULL and S = 0 for
 * no residual summaries (the summary arguments are as in
 * spruce_sparse_prefill_index_summaries).  A query row whose causal listed keys are all
 * padding (a left-padded position) writes zeros.
 */
int spruce_sparse_prefill_index_masked(
    const void* q, const int64_t qs[4],
    const void* k, const int64_t ks[4],
    const void* v, const int64_t vs[4],
    const int32_t* idx, const int64_t is[4], int64_t K,
    const uint8_t* key_valid, int64_t kvs,
    const int32_t* nodes, const int64_t ns[4], int64_t S,
    const void* sum_keys, const void* sum_values, const float* sum_log_counts, int sum_dtype,
    int64_t N, int64_t P,
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
    float scale, int dtype, int variant,
    void* out, const int64_t os[4],
    void* stream);

/*
 * The padded-list kernel with a general 4-D attention mask added to the
 * scores, as sparse_prefill_attention_forward does with any Transformers
 * mask (sparse/attention.py:223-229: scores scaled, future keys of the query
 * masked, then + attention_mask[b, :, q, key] for every listed key).
 *   amask  [B, Hm, Tq >= T, Tk >= T] with element strides ams (last 1),
 *          Hm = 1 (broadcast over heads) or Hq (one mask per query head);
 *   amask_dtype  SPRUCE_DTYPE_BF16 / F16 / F32: values added to the scaled
 *          score (0 attends, -inf or finfo.min gives no weight); U8: boolean,
 *          nonzero attends, zero gives no weight.
 * A query row none of whose listed causal keys survives the mask writes
 * zeros.  scale must be finite and nonzero (mask values are divided by it
 * to reach the unscaled scores' units).  Same launch shapes and arithmetic
 * as spruce_sparse_prefill_index otherwise.  No counterpart entry in the reference's kernels (its Triton
 * callback rejects attention masks, kernels/sparse_prefill.py:73-79); this is
 * the compute of its PyTorch path for masked prefill.
 */
int spruce_sparse_prefill_index_amask(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                      const void* v, const int64_t vs[4], const int32_t* idx, const int64_t is[4],
                                      int64_t K, const void* amask, const int64_t ams[4], int64_t Hm,
                                      int64_t Tq, int64_t Tk, int amask_dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                      int64_t T, int64_t D, float scale, int dtype, int variant, void* out,
                                      const int64_t os[4], void* stream);

/*
 * Residual-tree frontiers.  Replaces build_residual_summary_nodes /
 * residual_frontier_for_row (interfaces/residual_summaries.py:119-222): for
 * each row (b, l, g, q) of selected [B, L, G, Qb, K] int32 (element strides
 * ss[5], any order and duplicates; entries < 0 ignored), the maximal nodes of
 * the leaf-first binary tree over Qb leaves whose leaf ranges cover the
 * causal blocks [0, q] the row does not list, ascending by node ID.
 *   counts int32 [B*L*G*Qb]: frontier size per row, or -1 where the row lists
 *          an id > q (the reference raises ValueError there).
 *   out    int32 [B*L*G*Qb, S] contiguous with -1 padding, or NULL with S = 0
 *          to only count (call once to size S = max(counts), then again).
 * Qb up to about 250000 (tree bits in 64 KB of LDS).
 */
int spruce_residual_frontier(const int32_t* selected, const int64_t ss[5], int64_t B, int64_t L,
                             int64_t G, int64_t Qb, int64_t K, int32_t* counts, int32_t* out, int64_t S,
                             void* stream);

/* ------------------------------------------------------------------------
 * Selector front end.  These results are reproducible bit for bit: every
 * float is produced by a fixed sequence of IEEE single-precision operations
 * (documented in the library source) so the selected block indices can be
 * compared exactly with a CPU restatement.
 * ---------------------------------------------------------------------- */

/*
 * Block pooling of Q and K into per-64-token-block summaries.
 *   q [B, Hq, T, D] (strides qs) -> q_mean float32 [B, Hkv, ceil(T/64), D]:
 *     the query heads of each KV group averaged per token, then the block mean
 *     (replaces _group_avg_tokens + the prototype-0 mean of _proto_pool_seq,
 *     teacher/chunked_extract.py:75-80 and :27-72; the reference rounds each
 *     step to the model dtype, this computes in float32).
 *   k [B, Hkv, T, D] (strides ks) -> k_sum float32 [B, Hkv, ceil(T/64), 2, D]:
 *     prototype 0 = block mean (the leaf summary of sparse/summaries.py:52-142
 *     with all tokens valid), prototype 1 = per-dim block max.
 * Either input may be NULL to skip it.  D % 8 == 0.
 */
int spruce_selector_pool(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                         int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype,
                         float* q_mean, float* k_sum, void* stream);

/*
 * out[n][j] = sum_d x[n][d] * w[d][j] (float32, sequential fused multiply-add
 * over d).  x [N, D], w [D, P], out [N, P], all contiguous.
 * Replaces FlatGate.project_queries / project_keys (selector/gate.py:120-127).
 */
int spruce_gate_project(const float* x, const float* w, int64_t N, int64_t D, int64_t P, float* out,
                        void* stream);

/*
 * Two projections in one launch: outa = xa @ wa [Na, P], outb = xb @ wb
 * [Nb, P], both with the D x P shape and the arithmetic of
 * spruce_gate_project (identical results).  Replaces the pair
 * FlatGate.project_queries + project_keys of one layer (selector/gate.py:120-127).
 */
int spruce_gate_project2(const float* xa, const float* wa, int64_t Na, const float* xb, const float* wb,
                         int64_t Nb, int64_t D, int64_t P, float* outa, float* outb, void* stream);

/*
 * The projection of spruce_gate_project applied to prototype rows that sit in
 * several model-dtype buffers, written as one float32 table: level v's buffer
 * levels[v] holds [S, level_nodes[v], Pk, D] (contiguous, dtype bf16 / f16 /
 * f32, 8-byte aligned for 16-bit types, 16-byte for f32), and out
 * [S, N, Pk, P] (N = sum of level_nodes) takes the levels' nodes in order
 * (node IDs leaf-first for a key tree).  Every value is widened to float32
 * exactly, so the results equal spruce_gate_project's on a float32 copy of
 * the concatenated levels.  layout SPRUCE_KP_ROWS writes out as above;
 * SPRUCE_KP_INTERLEAVED writes [S, N, P/4, Pk, 4]: value (s, n, c, e) at
 * ((s*N + n)*(P/4) + e/4)*Pk*4 + c*4 + e%4, the key layout
 * spruce_tree_traverse reads fastest.  Replaces FlatGate.project_keys over the levels of
 * the key tree (selector/gate.py:124-127, called per level by
 * scripts/eval_tree_traversal.py:96) and, with one level,
 * FlatGate.project_queries (:120-122) on model-dtype prototypes.
 * Errors: 0 or more than 32 levels, D or P not multiples of 4, misaligned
 * buffers.
 */
int spruce_gate_project_levels(const void* const* levels, const int64_t* level_nodes, int64_t nlevels, int64_t S,
                               int64_t Pk, int64_t D, int dtype, const float* w, int64_t P, float* out, int layout,
                               void* stream);

/*
 * MaxSim block scores: scores[s][i][j] = max over prototype pairs (a, c) of
 * qp[s][i][a] . kp[s][j][c], divided by div (= sqrt(P)).  causal = 1: only
 * j <= i is computed and j > i is written as -inf; causal = 2 with Qb == Kb:
 * only j <= i is computed and the entries j > i are unspecified (for a
 * consumer such as spruce_causal_topk that reads only j <= i); causal = 0: all.
 * qp [S, Qb, Pq, P], kp [S, Kb, Pk, P], scores [S, Qb, Kb] contiguous.
 * Replaces FlatGate.forward (selector/gate.py:29-101) plus the causal mask of
 * selector/recall.py:26-35.
 */
int spruce_gate_scores(const float* qp, const float* kp, int64_t S, int64_t Qb, int64_t Kb,
                       int64_t Pq, int64_t Pk, int64_t P, float div, int causal, float* scores,
                       void* stream);

/*
 * Causal top-k block selection per row: the k largest of scores[r][i][0..i]
 * (ties to the lower block index, the stable descending argsort of
 * selector/baselines.py:59-62), written ascending into out[r][i][0..k) with
 * -1 padding when the row has fewer than k causal blocks -- the
 * selected_blocks row layout (interfaces/selected_blocks_spec.md).
 * scores [R, Qb, Kb] float32, out [R, Qb, k] int32, contiguous; Kb <= 8192.
 */
int spruce_causal_topk(const float* scores, int64_t R, int64_t Qb, int64_t Kb, int64_t k, int32_t* out,
                       void* stream);

/*
 * Block pooling and the gate projection in one launch: the values of
 * spruce_selector_pool (query group-and-block mean, key block mean and max;
 * teacher/chunked_extract.py:27-80 and :75-80 with the builder's max summary)
 * followed by spruce_gate_project2 (selector/gate.py:120-127), without the
 * pooled summaries in memory.
 *   q [B, Hq, T, 128], k [B, Hkv, T, 128] (any strides, contiguous last dim,
 *   16-byte aligned rows, each (batch, KV group) slice within 2^31 bytes),
 *   bf16 or f16, Hq / Hkv <= 8; wq, wk [128, 128] float32; P = 128.
 *   qp [B, Hkv, nb, 128] and kp [B, Hkv, nb, 2, 128] float32 (nb = ceil(T / 64);
 *   kp's [.., 0, :] is the projected block mean, [.., 1, :] the projected max).
 */
int spruce_selector_pool_project(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype,
                                 const float* wq, const float* wk, int64_t P, float* qp, float* kp,
                                 void* stream);

/*
 * The whole flat selector in two launches: the reference's flat route
 * (scripts/eval_gate.py:70-72) -- pooled block features
 * (teacher/chunked_extract.py:27-80), FlatGate MaxSim scoring
 * (selector/gate.py:29-101), causal mask and top-k (selector/recall.py:26-35,
 * ties per selector/baselines.py:59-62) -- with the selected blocks identical
 * to spruce_selector_pool -> spruce_gate_project2 -> spruce_gate_scores ->
 * spruce_causal_topk on the same inputs.
 *   q [B, Hq, T, 128], k [B, Hkv, T, 128] (any strides, contiguous last dim,
 *   16-byte aligned rows), bf16 or f16; wq, wk [128, 128] float32; P = 128;
 *   div the score divisor (sqrt(P) in the reference); out [B, Hkv, nb, top_k]
 *   int32 (nb = ceil(T / 64) <= 1024, Hq / Hkv <= 8).
 *   workspace: spruce_select_flat_workspace_bytes(B, Hkv, T, P) bytes, 16-byte
 *   aligned (the projected block keys).
 * spruce_select_flat_supported says whether a shape is covered (1) or not (0).
 */
int spruce_select_flat_supported(int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype, int64_t P);
int64_t spruce_select_flat_workspace_bytes(int64_t B, int64_t Hkv, int64_t T, int64_t P);
int spruce_select_flat(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype, const float* wq,
                       const float* wk, int64_t P, float div, int64_t top_k, void* workspace,
                       int64_t workspace_bytes, int32_t* out, void* stream);

/*
 * One parent level of the key-axis prototype tree.  Replaces
 * _merge_level_prototypes inside build_key_tree (selector/tree.py:79-145).
 *   child  [S, n, P, D] contiguous, S = layers * KV groups, dtype bf16/f16/f32.
 *   parent [S, ceil(n/radix), P, D] contiguous, same dtype.
 * Parent j covers children [j*radix, min((j+1)*radix, n)).  Prototype 0 is
 * rnd(rnd(sum of the children's prototype 0) / count) (float32 sum in child
 * order, rnd = round to the model dtype); prototypes 1..P-1 are the child
 * prototypes farthest from it in float32 squared L2, farthest first, ties to
 * the lower candidate (child-major, prototype-minor).  radix*P <= 64, D <= 256.
 */
int spruce_tree_merge_level(const void* child, int64_t S, int64_t n, int64_t P, int64_t D, int64_t radix,
                            int dtype, void* parent, void* stream);

/*
 * `levels` consecutive parent levels of the key-axis prototype tree from one
 * call, each level formed as spruce_tree_merge_level forms it (identical
 * results).  Replaces build_key_tree's level loop (selector/tree.py:116-145).
 *   child      [S, n, P, D] contiguous device tensor.
 *   parents    host array of `levels` device pointers; parents[v] is level
 *              v + 1 above the child, [S, n_{v+1}, P, D] contiguous, with
 *              n_{v+1} = ceil(n_v / radix) and n_0 = n.
 * Wide levels get one launch each (one wavefront per parent); once a level
 * has no more parents than fit as wavefronts of one workgroup in 64 KB of
 * LDS (at most 16), it and every level above it share one launch, one
 * workgroup per slab.  1 <= levels <= 32; other limits as
 * spruce_tree_merge_level.
 */
int spruce_tree_merge_levels(const void* child, int64_t S, int64_t n, int64_t P, int64_t D, int64_t radix,
                             int dtype, void* const* parents, int64_t levels, void* stream);

/*
 * Top-down beam traversal of the key tree.  Replaces traverse_to_leaf_ids
 * (scripts/eval_tree_traversal.py:59-113).
 *   qp  [S, qb, Pq, p] float32: projected query prototypes (FlatGate.project_queries).
 *   kp  [S, N, Pk, p] float32: projected key prototypes of every tree node,
 *       node IDs leaf-first (level v node i at sum of the lower level counts
 *       + i; level counts kb, ceil(kb/radix), ..., 1).
 *   out [S, qb, C] int32 leaf block IDs, score descending (ties to the lower
 *       node), -1 where no valid candidate was left; C must equal the final
 *       beam width min over levels of (beam, width*radix, level nodes).
 * At each level the children of the beam are scored with the MaxSim of
 * spruce_gate_candidate_scores; a child is valid when it exists and its first
 * leaf is <= the query block.  beam*radix <= 64, Pq <= 16, Pk <= 64,
 * p % 4 == 0 and Pq*p <= 8192.  Node choices are bit-reproducible.
 * layout: kp as SPRUCE_KP_ROWS (above) or SPRUCE_KP_INTERLEAVED
 * ([S, N, p/4, Pk, 4], written by spruce_gate_project_levels); the results
 * are identical, the interleaved table is read with 8x fewer cache lines per
 * load instruction.
 */
int spruce_tree_traverse(const float* qp, const float* kp, int64_t S, int64_t qb, int64_t kb, int64_t Pq,
                         int64_t Pk, int64_t p, int64_t radix, int64_t beam, float div, int32_t* out, int64_t C,
                         int layout, void* stream);

/*
 * MaxSim scores of per-row candidate nodes.  Replaces
 * FlatGate.score_projected_candidates (selector/gate.py:129-166).
 *   qp [S, qb, Pq, p], kp [S, N, Pk, p] float32; ids [S, qb, C] int32
 *   (clamped to [0, N-1] as the reference does); out [S, qb, C] float32 =
 *   max over key prototypes c of (max over query prototypes a of the fmaf
 *   chain q_a . k_c over p), divided by div.
 */
int spruce_gate_candidate_scores(const float* qp, const float* kp, const int32_t* ids, int64_t S, int64_t qb,
                                 int64_t N, int64_t C, int64_t Pq, int64_t Pk, int64_t p, float div, float* out,
                                 void* stream);

/* ------------------------------------------------------------------------
 * Teacher target extraction.
 * ---------------------------------------------------------------------- */

/* Schedules of the teacher block mass (a row's mass needs its final softmax
 * denominator before its rows are summed):
 *   SPRUCE_TEACHER_SCRATCH  single pass; each row's per-key-block partial
 *                           sum and reference point (8 bytes per row and key
 *                           block) go to the workspace, while they take at
 *                           most 4 GiB (T <= 32K at 28 query heads);
 *   SPRUCE_TEACHER_TWO_PASS row statistics, then QK^T again for the mass.
 * SPRUCE_TEACHER_AUTO takes the single pass when it applies and the
 * workspace holds it.  Both write per-half tile partials [B, Hq, 2, Qb, Qb]
 * float32 to the workspace and add the two halves into mass. */
#define SPRUCE_TEACHER_AUTO 0
#define SPRUCE_TEACHER_SCRATCH 1
#define SPRUCE_TEACHER_TWO_PASS 2

/* Device workspace of spruce_teacher_block_mass, Qb = ceil(T/64).
 * _min: the two-pass schedule -- row statistics [B, Hq, T, 2] plus the
 *   tile partials.
 * spruce_teacher_workspace_bytes: enough for every schedule (the scratch
 *   schedule's partials included while they take at most 4 GiB).
 * spruce_teacher_schedule_workspace_bytes: what one schedule needs.
 * spruce_teacher_schedule: the schedule SPRUCE_TEACHER_AUTO takes for this
 *   shape given workspace_bytes of workspace (SIZE_MAX: unlimited), or
 *   SPRUCE_EINVAL for an invalid shape.
 * These are the ABI's own sizing helpers (no reference counterpart). */
size_t spruce_teacher_workspace_bytes(int64_t B, int64_t Hq, int64_t T);
size_t spruce_teacher_workspace_bytes_min(int64_t B, int64_t Hq, int64_t T);
size_t spruce_teacher_schedule_workspace_bytes(int64_t B, int64_t Hq, int64_t T, int schedule);
int spruce_teacher_schedule(int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, size_t workspace_bytes);

/*
 * Dense causal softmax attention reduced to block probability mass without
 * forming the [T, T] matrix: mass[b][h][I][J] = sum over query rows i of
 * block I and keys j <= i of block J of softmax_j(q_i . k_j * scale), with
 * query head h reading KV head h / (Hq/Hkv); 0 for J > I.
 * Replaces chunked_pool (teacher/chunked_extract.py:91-131) with the GQA
 * repetition of _repeat_kv (:83-88) folded in.
 *   q [B, Hq, T, D], k [B, Hkv, T, D] (strides as for the attention entry
 *   points), mass float32 [B, Hq, Qb, Qb] contiguous, D in {64, 128}.
 * Rows of mass sum to the number of real query rows of the block (64).
 * The _schedule form takes one of the SPRUCE_TEACHER_* schedules (an
 * inapplicable one is SPRUCE_EINVAL); the plain form is SPRUCE_TEACHER_AUTO.
 */
int spruce_teacher_block_mass(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, float scale,
                              int dtype, float* mass, float* workspace, size_t workspace_bytes,
                              void* stream);
int spruce_teacher_block_mass_schedule(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, float scale,
                                       int dtype, float* mass, float* workspace, size_t workspace_bytes,
                                       int schedule, void* stream);

/*
 * Teacher targets from block mass (load_teacher, selector/targets.py:104-121,
 * and the top-k targets of selector/loss.py:34-46): per (b, KV head g, query
 * block i) the mean of mass over the group's query heads, zero above the
 * diagonal, row_mass = its row sum, target = mass / max(row_mass, eps), and
 * topk = the k causal blocks with the largest target, ordered by target
 * descending (ties to the lower block index), -1 padding for short rows.
 *   mass [B, Hq, Qb, Kb] -> target [B, Hkv, Qb, Kb], row_mass [B, Hkv, Qb],
 *   topk int32 [B, Hkv, Qb, k]; all contiguous; 1 <= k <= 64, Kb <= 8192.
 */
int spruce_teacher_targets(const float* mass, int64_t B, int64_t Hq, int64_t Hkv, int64_t Qb, int64_t Kb,
                           int64_t k, float eps, float* target, float* row_mass, int32_t* topk,
                           void* stream);

/*
 * The first half of spruce_teacher_targets alone: group_mass = the mean of
 * mass over each KV group's query heads, zero above the diagonal, and
 * row_mass its row sum, without normalisation (load_teacher with
 * defer_normalization=True, selector/targets.py:104-113).
 *   mass [B, Hq, Qb, Kb] -> group_mass [B, Hkv, Qb, Kb], row_mass [B, Hkv, Qb];
 *   all contiguous; Kb <= 8192.
 */
int spruce_teacher_group_mass(const float* mass, int64_t B, int64_t Hq, int64_t Hkv, int64_t Qb, int64_t Kb,
                              float* group_mass, float* row_mass, void* stream);

/*
 * Selector prototype features in the model dtype.  Replaces _proto_pool_seq
 * (teacher/chunked_extract.py:27-72) applied to _group_avg_tokens (:75-80):
 * x [B, H, L, D] (strided, element strides xs) is averaged over the H/G heads
 * of each group per token (G == H: no averaging), then per block of `block`
 * tokens prototype 0 is the mean of the real rows and prototypes 1..k,
 * k = min(P-1, block), are the k rows farthest from it in float32 squared L2
 * (farthest first, ties to the lower row); slots past the real rows hold the
 * mean.  out [B, G, ceil(L/block), P, D] contiguous, x's dtype.
 * Limits: D <= 128, 1 <= block <= 64, 1 <= P <= 65.  Deterministic (fixed
 * float32 operation order).
 */
int spruce_proto_pool(const void* x, const int64_t xs[4], int64_t B, int64_t H, int64_t L, int64_t D,
                      int64_t G, int64_t block, int64_t P, int dtype, void* out, void* stream);

/*
 * Query and key prototypes of the same blocks in one launch: out_q equals
 * spruce_proto_pool(q, ..., H = Hq, G = Hkv, ...) and out_k equals
 * spruce_proto_pool(k, ..., H = G = Hkv, ...) (teacher/chunked_extract.py:27-80
 * on both sides, as the capture hook :145-147 calls them).  16-bit q and k
 * with a contiguous last dim and 16-byte aligned rows, D a multiple of 8 up to
 * 128, Hq / Hkv <= 8, 1 <= block <= 64, 1 <= P <= 65.
 */
int spruce_proto_pool_qk(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t L, int64_t D, int64_t block, int64_t P, int dtype,
                         void* out_q, void* out_k, void* stream);

/*
 * Per-token group average, x [B, H, L, D] -> out [B, G, L, D] contiguous, x's
 * dtype.  Replaces _group_avg_tokens (teacher/chunked_extract.py:75-80).
 */
int spruce_group_avg_tokens(const void* x, const int64_t xs[4], int64_t B, int64_t H, int64_t L, int64_t D,
                            int64_t G, int dtype, void* out, void* stream);

/*
 * Residual-tree K/V summary table.  Replaces build_kv_summary_table
 * (sparse/summaries.py:52-142): for each of R token ranges [start, end)
 * (range_starts / range_ends, int64 device arrays, one per tree node and
 * prototype as _prototype_token_ranges builds them, :29-49), the float32 mean
 * of the valid K and V rows and the valid-token count.
 *   k, v        [B, Hkv, T, D] strided (element strides ks, vs).
 *   valid       uint8 [B, T] key-padding mask (nonzero = real token) or NULL.
 *   keys/values float32 [B, Hkv, R, D]; counts, log_counts float32 [B, R];
 *               mean = sum / max(count, 1); log_counts = -inf where count = 0.
 *   workspace   >= spruce_kv_summary_workspace_bytes(B, Hkv, T, D) bytes,
 *               256-byte aligned (per-64-token chunk sums).
 * Range bounds are clamped to [0, T] on the device.
 */
size_t spruce_kv_summary_workspace_bytes(int64_t B, int64_t Hkv, int64_t T, int64_t D);
int spruce_kv_summary(const void* k, const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B,
                      int64_t Hkv, int64_t T, int64_t D, int dtype, const uint8_t* valid,
                      const int64_t* range_starts, const int64_t* range_ends, int64_t R, float* keys,
                      float* values, float* counts, float* log_counts, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * spruce_kv_summary without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  The workspace is a library-held static device buffer of
 * SPRUCE_KV_SUMMARY_NOALLOC_MAX_BYTES (64 MiB) per GPU, held from the first
 * use of the library's summary kernels on that GPU until the process ends;
 * shapes with spruce_kv_summary_workspace_bytes(B, Hkv, T, D) above it (for
 * example B * Hkv * T > 4 * 65536 at D = 128) return SPRUCE_EINVAL.
 * The current device must be the device of `stream`.  Every call on one GPU
 * shares that buffer, so the calls on one GPU are ordered: each call's
 * kernels wait (hipStreamWaitEvent on a per-device event, created on the
 * device's first call) for the previous call's, whatever stream either was
 * issued on, and calls from several host threads enter one at a time.  A call
 * issued under stream capture is not ordered this way (the event would tie the
 * graph to uncaptured work): replays of captured calls that may overlap each
 * other or uncaptured calls on the same GPU must be serialised by the caller.
 * Results are identical to spruce_kv_summary's.
 */
#define SPRUCE_KV_SUMMARY_NOALLOC_MAX_BYTES (64u << 20)
int spruce_kv_summary_noalloc(const void* k, const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B,
                              int64_t Hkv, int64_t T, int64_t D, int dtype, const uint8_t* valid,
                              const int64_t* range_starts, const int64_t* range_ends, int64_t R, float* keys,
                              float* values, float* counts, float* log_counts, void* stream);

/*
 * Packs compact traversal IDs into selected_blocks rows.  Replaces
 * selected_ids_to_blocks (scripts/export_selected_blocks.py:79-175), same
 * policy: forced sink blocks [0, min(sink_blocks, key_blocks)) strictly before
 * the local window, then the smallest distinct IDs in
 * [sink, min(q - local_window, key_blocks)) up to the remaining budget, then
 * the local window q-local_window..q (ids >= 0); ascending, PAD -1.
 *   ids  [R, C] contiguous, int32 (id_bytes 4) or int64 (id_bytes 8), rows
 *        ordered (layer, kv head, query block) so q = row % qb; any value
 *        allowed (out-of-range IDs are ignored, duplicates count once).
 *   out  int32 [R, out_cols] contiguous; out_cols must equal
 *        min(k_selected, C + min(sink_blocks, key_blocks) + local_window + 1).
 * Errors: k_selected < local_window + 1 + sink_blocks, key_blocks < 1 or
 * > 65536, negative local_window/sink_blocks.
 */
int spruce_pack_selected_ids(const void* ids, int id_bytes, int64_t R, int64_t qb, int64_t C,
                             int64_t key_blocks, int64_t k_selected, int64_t local_window,
                             int64_t sink_blocks, int32_t* out, int64_t out_cols, void* stream);

/*
 * Packs a boolean route mask into selected_blocks rows.  Replaces
 * selected_mask_to_blocks (scripts/export_selected_blocks.py:37-76): the
 * local window q-local_window..min(q, kb-1) is forced, and the first causal
 * non-local columns of the row fill the rest of k_selected; ascending, PAD -1.
 *   mask uint8 [R, kb] contiguous (nonzero = selected), q = row % qb.
 *   out  int32 [R, out_cols], out_cols = min(k_selected, kb).
 */
int spruce_pack_selected_mask(const uint8_t* mask, int64_t R, int64_t qb, int64_t kb, int64_t k_selected,
                              int64_t local_window, int32_t* out, int64_t out_cols, void* stream);

/*
 * Launch configuration the attention entry points use for a shape, as JSON:
 * {"variant":..,"best_config":{..}}.  Replaces kernel_runtime_metadata
 * (kernels/seerattention_direct_index_triton.py:430-447).
 */
int spruce_kernel_metadata(int variant, int64_t Hq, int64_t Hkv, int64_t D,
                           char* json, size_t n);

#ifdef __cplusplus
}
#endif

#endif /* SPRUCE_HIP_H */
