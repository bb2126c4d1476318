// spruce_sparse_prefill_index_amask: padded direct-index block lists with a
// general 4-D attention mask added to the scores (the masked prefill of
// sparse/attention.py:223-229).
#include <cmath>

#include "attention_impl.h"

using namespace spruce;

extern "C" int spruce_sparse_prefill_index_amask(
    const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], const void* v,
    const int64_t vs[4], const int32_t* idx, const int64_t is[4], int64_t K, const void* amask,
    const int64_t ams[4], int64_t Hm, int64_t Tq, int64_t Tk, int amask_dtype, int64_t B, int64_t Hq,
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
  SPRUCE_REQUIRE(amask != nullptr && ams != nullptr, "the attention mask must be a non-null device pointer");
  SPRUCE_REQUIRE(Hm == 1 || Hm == Hq, "the attention mask must have 1 or Hq (%lld) heads, got %lld",
                 (long long)Hq, (long long)Hm);
  SPRUCE_REQUIRE(Tq >= T && Tk >= T, "the attention mask [.., %lld, %lld] must cover %lld query and key tokens",
                 (long long)Tq, (long long)Tk, (long long)T);
  SPRUCE_REQUIRE(ams[3] == 1, "the attention mask must have a contiguous last dimension");
  SPRUCE_REQUIRE(ams[0] >= 0 && ams[1] >= 0 && ams[2] >= 0, "negative attention mask strides");
  SPRUCE_REQUIRE(Tk < ((int64_t)1 << 30), "attention mask too wide");
  SPRUCE_REQUIRE(amask_dtype == SPRUCE_DTYPE_BF16 || amask_dtype == SPRUCE_DTYPE_F16 ||
                     amask_dtype == SPRUCE_DTYPE_F32 || amask_dtype == SPRUCE_DTYPE_U8,
                 "unsupported attention mask dtype code %d", amask_dtype);
  const int eb = amask_dtype == SPRUCE_DTYPE_F32 ? 4 : (amask_dtype == SPRUCE_DTYPE_U8 ? 1 : 2);
  p.idx = idx;
  for (int i = 0; i < 4; ++i) {
    p.is[i] = is[i];
    p.ams[i] = ams[i];
  }
  p.K = (int)K;
  p.amask = amask;
  p.amask_dtype = amask_dtype;
  p.amask_heads = (int)Hm;
  // Groups of 4 keys start at multiples of 4 elements within a row, so one
  // aligned load covers a group when the base and the row strides are
  // multiples of 4 elements.
  p.amask_vec = ((uintptr_t)amask % (uintptr_t)(4 * eb)) == 0 && ams[0] % 4 == 0 && (Hm == 1 || ams[1] % 4 == 0) &&
                ams[2] % 4 == 0;
  // Whole 16-byte row pieces: the base and every row start 16-byte aligned
  // (a block's 64 keys start at a multiple of 64 elements).
  p.amask_rows16 = ((uintptr_t)amask % 16) == 0 && (ams[0] * eb) % 16 == 0 && (Hm == 1 || (ams[1] * eb) % 16 == 0) &&
                   (ams[2] * eb) % 16 == 0;
  p.amask_tk = (int)Tk;
  // Mask values are brought to the unscaled scores' units (one multiply
  // before the scale's FMA), so the scale must be finite and nonzero.
  p.amask_mul = 1.4426950408889634f / p.cs;
  SPRUCE_REQUIRE(std::isfinite(p.amask_mul) && std::isfinite(p.cs),
                 "the attention mask entry needs a finite nonzero scale, got %g", (double)scale);
  return launch_attention<kModePadded, false, false, true>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}
