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
  split_small_grid(p, shape, variant);
  SPRUCE_REQUIRE(idx != nullptr && is != nullptr, "indices must be a non-null device pointer");
  SPRUCE_REQUIRE(K >= 0 && K < (int64_t)1 << 30, "invalid index row width K=%lld", (long long)K);
  p.idx = idx;
  for (int i = 0; i < 4; ++i) p.is[i] = is[i];
  p.K = (int)K;
  return launch_attention<kModePadded>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}

namespace {

// Summary-table arguments of the residual-summary entry points.
int set_summaries(AttnParams& p, const int32_t* nodes, const int64_t ns[4], int64_t S, const void* sum_keys,
                  const void* sum_values, const float* sum_log_counts, int sum_dtype, int dtype, int64_t N,
                  int64_t P) {
  SPRUCE_REQUIRE(ns != nullptr && S >= 0 && S < (int64_t)1 << 24, "invalid summary node rows (S=%lld)",
                 (long long)S);
  SPRUCE_REQUIRE(nodes != nullptr || S == 0, "nodes must be a non-null device pointer");
  SPRUCE_REQUIRE(N >= 0 && N < (int64_t)1 << 26, "invalid summary node count N=%lld", (long long)N);
  SPRUCE_REQUIRE(P >= 1 && P <= 64, "summary prototypes must be in [1, 64], got %lld", (long long)P);
  SPRUCE_REQUIRE(N == 0 || (sum_keys && sum_values && sum_log_counts),
                 "summary table pointers must be non-null");
  SPRUCE_REQUIRE(((uintptr_t)sum_keys % 16) == 0 && ((uintptr_t)sum_values % 16) == 0,
                 "summary keys/values must be 16-byte aligned");
  SPRUCE_REQUIRE(sum_dtype == SPRUCE_DTYPE_F32 || (sum_dtype == dtype && dtype != SPRUCE_DTYPE_F32),
                 "summary keys/values must be float32 or the 16-bit input dtype (code %d), got code %d", dtype,
                 sum_dtype);
  p.snode = nodes;
  for (int i = 0; i < 4; ++i) p.sns[i] = ns[i];
  p.S = (int)S;
  p.N = (int)N;
  p.P = (int)P;
  p.skey = sum_keys;
  p.sval = sum_values;
  p.sum16 = sum_dtype != SPRUCE_DTYPE_F32;
  p.slog = sum_log_counts;
  p.sbias = 1.4426950408889634f / p.cs;
  return SPRUCE_OK;
}

}  // namespace

// spruce_sparse_prefill_index_summaries: the same padded lists plus the
// residual-summary keys of sparse/attention.py:226-265 (one extra softmax
// entry per listed tree node and prototype, biased by log(count)).
extern "C" int spruce_sparse_prefill_index_summaries(
    const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], const void* v,
    const int64_t vs[4], const int32_t* idx, const int64_t is[4], int64_t K, const int32_t* nodes,
    const int64_t ns[4], int64_t S, const void* sum_keys, const void* sum_values,
    const float* sum_log_counts, int sum_dtype, int64_t N, int64_t P, int64_t B, int64_t Hq, int64_t Hkv,
    int64_t T, int64_t D, float scale, int dtype, int variant, void* out, const int64_t os[4], void* stream) {
  AttnParams p;
  LaunchShape shape;
  int rc = prepare_attention(p, q, qs, k, ks, v, vs, B, Hq, Hkv, T, D, scale, dtype, variant, out, os,
                             shape);
  if (rc) return rc;
  split_small_grid(p, shape, variant);
  SPRUCE_REQUIRE(idx != nullptr && is != nullptr, "indices must be a non-null device pointer");
  SPRUCE_REQUIRE(K >= 0 && K < (int64_t)1 << 30, "invalid index row width K=%lld", (long long)K);
  rc = set_summaries(p, nodes, ns, S, sum_keys, sum_values, sum_log_counts, sum_dtype, dtype, N, P);
  if (rc) return rc;
  p.idx = idx;
  for (int i = 0; i < 4; ++i) p.is[i] = is[i];
  p.K = (int)K;
  return launch_attention<kModePadded, true>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}

// spruce_sparse_prefill_index_masked: padded lists with a key-padding mask
// (the padded-batch prefill of sparse/attention.py:147-150,225-229, where the
// decoder mask is causal plus key validity), optionally with residual
// summaries (nodes == NULL and S == 0 for none).
extern "C" int spruce_sparse_prefill_index_masked(
    const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], const void* v,
    const int64_t vs[4], const int32_t* idx, const int64_t is[4], int64_t K, const uint8_t* key_valid,
    int64_t kvs, const int32_t* nodes, const int64_t ns[4], int64_t S, const void* sum_keys,
    const void* sum_values, const float* sum_log_counts, int sum_dtype, int64_t N, int64_t P, int64_t B, int64_t Hq,
    int64_t Hkv, int64_t T, int64_t D, float scale, int dtype, int variant, void* out, const int64_t os[4],
    void* stream) {
  AttnParams p;
  LaunchShape shape;
  int rc = prepare_attention(p, q, qs, k, ks, v, vs, B, Hq, Hkv, T, D, scale, dtype, variant, out, os,
                             shape);
  if (rc) return rc;
  split_small_grid(p, shape, variant);
  SPRUCE_REQUIRE(idx != nullptr && is != nullptr, "indices must be a non-null device pointer");
  SPRUCE_REQUIRE(K >= 0 && K < (int64_t)1 << 30, "invalid index row width K=%lld", (long long)K);
  SPRUCE_REQUIRE(key_valid != nullptr, "key_valid must be a non-null device pointer");
  SPRUCE_REQUIRE(kvs >= T, "key_valid batch stride (%lld) must be at least T (%lld)", (long long)kvs,
                 (long long)T);
  p.idx = idx;
  for (int i = 0; i < 4; ++i) p.is[i] = is[i];
  p.K = (int)K;
  p.kvalid = key_valid;
  p.kvs = kvs;
  const bool summaries = S > 0;
  if (summaries) {
    rc = set_summaries(p, nodes, ns, S, sum_keys, sum_values, sum_log_counts, sum_dtype, dtype, N, P);
    if (rc) return rc;
    return launch_attention<kModePadded, true, true>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
  }
  return launch_attention<kModePadded, false, true>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}
