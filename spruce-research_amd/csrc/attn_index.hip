// spruce_sparse_prefill_index: padded direct-index block lists
// ([B, Hkv, Qb, K] int32, -1 padding), the layout of
// interfaces/selected_blocks_spec.md consumed by
// kernels/seerattention_direct_index_triton.py:339-416.
#include "attention_impl.h"

using namespace spruce;

extern "C" int spruce_sparse_prefill_index(
    const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], const void* v,
    const int64_t vs[4], const int32_t* idx, const int64_t is[4], int64_t K, int64_t B, int64_t Hq,
    int64_t Hkv, int64_t T, int64_t D, float scale, int dtype, int variant, void* out,
    const int64_t os[4], void* stream) {
  AttnParams p;
  LaunchShape shape;
  int rc = prepare_attention(p, q, qs, k, ks, v, vs, B, Hq, Hkv, T, D, scale, dtype, variant, out, os,
                             shape);
  if (rc) return rc;
  SPRUCE_REQUIRE(idx != nullptr && is != nullptr, "indices must be a non-null device pointer");
  SPRUCE_REQUIRE(K >= 0 && K < (int64_t)1 << 30, "invalid index row width K=%lld", (long long)K);
  p.idx = idx;
  for (int i = 0; i < 4; ++i) p.is[i] = is[i];
  p.K = (int)K;
  return launch_attention<kModePadded>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}
