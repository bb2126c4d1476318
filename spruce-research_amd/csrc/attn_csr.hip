// spruce_sparse_prefill_csr: variable-length (CSR) block lists, one row per
// (batch, KV head, query block).
#include "attention_impl.h"

using namespace spruce;

extern "C" int spruce_sparse_prefill_csr(
    const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], const void* v,
    const int64_t vs[4], const int32_t* indptr, const int32_t* indices, int64_t nnz, const int32_t* row_order,
    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, float scale, int dtype, int variant,
    void* out, const int64_t os[4], void* stream) {
  AttnParams p;
  LaunchShape shape;
  int rc = prepare_attention(p, q, qs, k, ks, v, vs, B, Hq, Hkv, T, D, scale, dtype, variant, out, os,
                             shape);
  if (rc) return rc;
  split_small_grid(p, shape, variant);
  SPRUCE_REQUIRE(nnz >= 0 && nnz < ((int64_t)1 << 31), "invalid nnz %lld", (long long)nnz);
  // With no entries (every row empty) indices is never read and may be null.
  SPRUCE_REQUIRE(indptr != nullptr && (indices != nullptr || nnz == 0), "indptr and indices must be non-null");
  p.indptr = indptr;
  p.nnz = (int)nnz;
  p.indices = indices;
  p.row_order = row_order;
  return launch_attention<kModeCsr>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}
