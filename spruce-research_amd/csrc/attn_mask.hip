// spruce_sparse_prefill_mask: boolean block mask [B, Hm, Qb, >=Qb], the layout
// produced by selected_blocks_to_block_mask (kernels/sparse_prefill.py:16-39)
// and consumed by block_sparse_triton (kernels/seerattention_triton.py:71-90).
#include "attention_impl.h"

using namespace spruce;

extern "C" int spruce_sparse_prefill_mask(
    const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], const void* v,
    const int64_t vs[4], const uint8_t* mask, const int64_t ms[4], int64_t Hm, int64_t B, int64_t Hq,
    int64_t Hkv, int64_t T, int64_t D, float scale, int dtype, int variant, void* out,
    const int64_t os[4], void* stream) {
  AttnParams p;
  LaunchShape shape;
  int rc = prepare_attention(p, q, qs, k, ks, v, vs, B, Hq, Hkv, T, D, scale, dtype, variant, out, os,
                             shape);
  if (rc) return rc;
  split_small_grid(p, shape, variant);
  SPRUCE_REQUIRE(mask != nullptr && ms != nullptr, "mask must be a non-null device pointer");
  SPRUCE_REQUIRE(Hm == Hq || Hm == Hkv, "mask heads (%lld) must equal query heads (%lld) or KV heads (%lld)",
                 (long long)Hm, (long long)Hq, (long long)Hkv);
  p.mask = mask;
  for (int i = 0; i < 4; ++i) p.ms[i] = ms[i];
  p.mask_per_qhead = (Hm == Hq && Hq != Hkv) ? 1 : 0;
  return launch_attention<kModeMask>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);
}
