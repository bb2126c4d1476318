// spruce_causal_prefill: dense causal GQA prefill (every key block 0..qb of
// every row, in order), optionally emitting the selector features of the
// reference's capture hooks as a by-product of the same pass
// (teacher/chunked_extract.py:163-180 `_capture_features`: group-averaged
// queries and the key prototypes of `_proto_pool_seq`, :27-80).
#include "attention_impl.h"

using namespace spruce;

namespace {

template <int D, typename TIn, bool F16>
int launch_capture(const AttnParams& p, hipStream_t stream) {
  if (p.tpp < 8) return launch_attention_t<D, 8, TIn, F16, kModeCausal, false, true, kUseProducer>(p, stream);
  return launch_attention_t<D, 8, TIn, F16, kModeCausal, false, true>(p, stream);
}

}  // namespace

extern "C" int spruce_causal_prefill(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                     const void* v, const int64_t vs[4], int64_t B, int64_t Hq, int64_t Hkv,
                                     int64_t T, int64_t D, float scale, int dtype, void* out, const int64_t os[4],
                                     void* q_grouped, void* k_protos, int64_t P, void* stream) {
  AttnParams p;
  LaunchShape shape;
  int rc = prepare_attention(p, q, qs, k, ks, v, vs, B, Hq, Hkv, T, D, scale, dtype, SPRUCE_VARIANT_TILED_GQA, out,
                             os, shape);
  if (rc) return rc;
  if (q_grouped == nullptr && k_protos == nullptr)
    return launch_attention<kModeCausal>(p, (int)D, dtype, shape.waves, (hipStream_t)stream);

  SPRUCE_REQUIRE(q_grouped != nullptr && k_protos != nullptr,
                 "feature capture needs both q_grouped and k_protos (or neither)");
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16,
                 "feature capture runs in the model dtype (bf16 or f16)");
  SPRUCE_REQUIRE(p.G <= 8, "feature capture supports at most 8 query heads per KV head, got %d", p.G);
  SPRUCE_REQUIRE(P >= 1 && P <= 65, "prototypes must be in [1, 65], got %lld", (long long)P);
  SPRUCE_REQUIRE(((uintptr_t)q_grouped % 16) == 0 && ((uintptr_t)k_protos % 16) == 0,
                 "q_grouped and k_protos must be 16-byte aligned");
  // One part per 32-row half when the G heads of a half fill a workgroup
  // (G > 4), else both halves in one part; 8-wave workgroups either way.
  p.parts = 2 * p.G > 8 ? 2 : 1;
  p.tpp = 2 * p.G / p.parts;
  p.P = (int)P;
  p.qgrp = q_grouped;
  p.kproto = k_protos;
  p.inv_rep = 1.0f / (float)p.G;
  p.prescale = 0;  // the group average reads the raw Q fragments
  const int64_t grid = ((int64_t)B * Hkv * p.Qb + 7) / 8 * 8 * p.parts;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "grid too large");
  if (D == 128)
    return dtype == SPRUCE_DTYPE_BF16 ? launch_capture<128, InBF16, false>(p, (hipStream_t)stream)
                                      : launch_capture<128, InF16, true>(p, (hipStream_t)stream);
  return dtype == SPRUCE_DTYPE_BF16 ? launch_capture<64, InBF16, false>(p, (hipStream_t)stream)
                                    : launch_capture<64, InF16, true>(p, (hipStream_t)stream);
}
