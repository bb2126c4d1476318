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

/* Element type of Q/K/V and of the attention output. */
#define SPRUCE_DTYPE_BF16 0
#define SPRUCE_DTYPE_F16 1
#define SPRUCE_DTYPE_F32 2

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
