// Error slot, version, launch-shape metadata and the argument checks shared by
// the attention entry points.
#include "attention_impl.h"

namespace spruce {

namespace {
thread_local char g_error[1024] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SPRUCE_OK;
}

static bool aligned_vec(const void* ptr, const int64_t s[4], int elem_bytes) {
  // 16-byte vector loads of 8 (16-bit) or 4 (fp32) elements along head_dim.
  const int64_t per16 = 16 / elem_bytes;
  if (reinterpret_cast<uintptr_t>(ptr) % 16) return false;
  for (int i = 0; i < 3; ++i)
    if (s[i] % per16) return false;
  return true;
}

int prepare_attention(AttnParams& p, const void* q, const int64_t qs[4], const void* k,
                      const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B,
                      int64_t Hq, int64_t Hkv, int64_t T, int64_t D, float scale, int dtype,
                      int variant, void* out, const int64_t os[4], LaunchShape& shape) {
  SPRUCE_REQUIRE(q && k && v && out, "q, k, v and out must be non-null device pointers");
  SPRUCE_REQUIRE(qs && ks && vs && os, "stride arrays must be non-null");
  SPRUCE_REQUIRE(D == 64 || D == 128, "kernel supports head_dim 64 or 128, got %lld", (long long)D);
  SPRUCE_REQUIRE(B >= 1 && T >= 1 && Hq >= 1 && Hkv >= 1, "B, T, Hq and Hkv must be positive");
  SPRUCE_REQUIRE(Hq % Hkv == 0, "query heads (%lld) must be divisible by KV heads (%lld)",
                 (long long)Hq, (long long)Hkv);
  SPRUCE_REQUIRE(Hq / Hkv <= 64, "at most 64 query heads per KV head are supported");
  SPRUCE_REQUIRE(T < (int64_t)1 << 30, "sequence length too large");
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  SPRUCE_REQUIRE(variant >= SPRUCE_VARIANT_SINGLE_HEAD && variant <= SPRUCE_VARIANT_TILED_GQA,
                 "unknown kernel variant %d", variant);
  SPRUCE_REQUIRE(qs[3] == 1 && ks[3] == 1 && vs[3] == 1 && os[3] == 1,
                 "q, k, v and out must have a contiguous final dimension");
  const int eb = dtype == SPRUCE_DTYPE_F32 ? 4 : 2;
  SPRUCE_REQUIRE(aligned_vec(q, qs, eb) && aligned_vec(k, ks, eb) && aligned_vec(v, vs, eb),
                 "q, k and v must be 16-byte aligned with strides that keep rows 16-byte aligned");
  SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(out) % 8 == 0 && os[0] % 4 == 0 && os[1] % 4 == 0 &&
                     os[2] % 4 == 0,
                 "out must be 8-byte aligned with strides that are multiples of 4 elements");
  // Buffer loads address a 64-token block (32-token tile) with 32-bit offsets.
  SPRUCE_REQUIRE(qs[2] * eb * 32 < ((int64_t)1 << 30) && os[2] * eb * 32 < ((int64_t)1 << 30) &&
                     ks[2] * eb * 64 < ((int64_t)1 << 30) && vs[2] * eb * 64 < ((int64_t)1 << 30),
                 "token strides too large");
  p = AttnParams{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = out;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = qs[i];
    p.ks[i] = ks[i];
    p.vs[i] = vs[i];
    p.os[i] = os[i];
  }
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.T = (int)T;
  p.G = (int)(Hq / Hkv);
  p.Qb = (int)((T + kBlock - 1) / kBlock);
  const float log2e = 1.4426950408889634f;
  p.prescale = variant == SPRUCE_VARIANT_SINGLE_HEAD_PRESCALE;
  p.cs = p.prescale ? 1.f : scale * log2e;
  p.qmul = scale * log2e;
  shape = choose_shape(variant, p.G);
  p.parts = shape.parts;
  p.tpp = shape.tpp;
  const int64_t grid = ((int64_t)B * Hkv * p.Qb + 7) / 8 * 8 * shape.parts;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "grid too large");
  return SPRUCE_OK;
}

}  // namespace spruce

using namespace spruce;

extern "C" int spruce_last_error(char* buf, size_t n) {
  const size_t len = strlen(g_error);
  if (buf && n) {
    const size_t c = len < n - 1 ? len : n - 1;
    memcpy(buf, g_error, c);
    buf[c] = 0;
  }
  return (int)len;
}

extern "C" const char* spruce_version(void) { return "spruce_hip 0.1 gfx950"; }

extern "C" int spruce_kernel_metadata(int variant, int64_t Hq, int64_t Hkv, int64_t D, char* json,
                                      size_t n) {
  static const char* names[] = {"single_head", "single_head_causal", "single_head_prescale",
                                "single_head_qtile", "tiled_gqa"};
  SPRUCE_REQUIRE(variant >= 0 && variant <= 4, "unknown kernel variant %d", variant);
  SPRUCE_REQUIRE(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "invalid head counts");
  SPRUCE_REQUIRE(D == 64 || D == 128, "head_dim must be 64 or 128");
  SPRUCE_REQUIRE(json && n, "json buffer required");
  const LaunchShape s = choose_shape(variant, (int)(Hq / Hkv));
  const int lds = 2 * (kBlock * ((int)D + 8) + (int)D * (kBlock + 8)) * 2;
  // best_config carries the reference's keys (kwargs, num_warps, num_stages,
  // num_ctas; kernels/seerattention_direct_index_triton.py:419-427) filled
  // with this launch: waves per workgroup, two K/V stages, one workgroup per
  // (row, part), the tile constants as kwargs; then the HIP-specific fields.
  const int w = snprintf(json, n,
                         "{\"variant\":\"%s\",\"best_config\":{"
                         "\"kwargs\":{\"QUERY_ROWS\":32,\"KEY_BLOCK\":64,\"TILES_PER_WORKGROUP\":%d,"
                         "\"WORKGROUPS_PER_ROW\":%d},\"num_warps\":%d,\"num_stages\":2,\"num_ctas\":1,"
                         "\"waves_per_workgroup\":%d,"
                         "\"workgroups_per_row\":%d,\"query_rows_per_wave\":32,\"key_block\":64,"
                         "\"lds_bytes\":%d,\"mfma\":\"v_mfma_f32_32x32x16\",\"prescale_q\":%s}}",
                         names[variant], s.tpp, s.parts, s.waves, s.waves, s.parts, lds,
                         variant == SPRUCE_VARIANT_SINGLE_HEAD_PRESCALE ? "true" : "false");
  return (w < 0 || (size_t)w >= n) ? set_error(SPRUCE_EINVAL, "json buffer too small") : SPRUCE_OK;
}
