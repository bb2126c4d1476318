/*
 * CPU oracle for the selector prototype features -- TEST INFRASTRUCTURE ONLY.
 * Used by tests/ as the checker of the HIP proto_pool / group_avg kernels.
 *
 * Restates, in the exact float32 operation order the HIP kernels use:
 *   oracle_group_avg   _group_avg_tokens (teacher/chunked_extract.py:75-80):
 *                      per token, rnd(sum_h x_h * fl(1/rep)) with the heads of
 *                      the group summed in order starting from 0.0f (torch's
 *                      GPU mean multiplies the float sum by the factor 1/n);
 *                      rep == 1 returns x unchanged.
 *   oracle_proto_pool  _proto_pool_seq (teacher/chunked_extract.py:27-72) over
 *                      the group-averaged rows: mean = rnd(rnd(sum_t a_t) / n)
 *                      over the block's n real rows (:47-48, the sum and the
 *                      division happen in the model dtype); float32 squared L2
 *                      distance to the mean (:55); the k = min(P-1, block)
 *                      farthest rows, farthest first, ties to the lower row
 *                      (torch.topk leaves tie order open), NaN largest
 *                      (:57-58); pad picks and extra slots hold the mean
 *                      (:64-70).
 * rnd() rounds to the model dtype, nearest even: dtype 0 bf16, 1 f16, 2 f32
 * (identity).  Inputs are float arrays holding model-dtype values.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Nearest-even rounding of a float32 to bfloat16 (8-bit significand). */
static float round_bf16(float x) {
  if (isnan(x)) return x;
  uint32_t u = bits_of(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return float_of(u & 0xffff0000u);
}

/* Nearest-even rounding of a float32 to IEEE binary16. */
static float round_f16(float x) {
  if (isnan(x) || isinf(x)) return x;
  const float ax = fabsf(x);
  if (ax < 0x1p-14f) {                        /* subnormal half: quantum 2^-24 */
    return nearbyintf(x * 0x1p24f) * 0x1p-24f;
  }
  uint32_t u = bits_of(x);
  u += 0xfffu + ((u >> 13) & 1u);             /* keep 10 fraction bits */
  const float r = float_of(u & 0xffffe000u);
  if (fabsf(r) > 65504.0f) return copysignf(INFINITY, x);
  return r;
}

static float rnd(float x, int dtype) {
  if (dtype == 0) return round_bf16(x);
  if (dtype == 1) return round_f16(x);
  return x;
}

/* Exported for the oracle's own tests: model-dtype rounding. */
void oracle_round(const float* x, int64_t n, int dtype, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = rnd(x[i], dtype);
}

/* x [B,H,L,D] -> out [B,G,L,D]. */
void oracle_group_avg(const float* x, int B, int H, int L, int D, int G, int dtype, float* out) {
  const int rep = H / G;
  const float inv = 1.0f / (float)rep;
  for (int b = 0; b < B; ++b)
    for (int g = 0; g < G; ++g)
      for (int t = 0; t < L; ++t)
        for (int d = 0; d < D; ++d) {
          const float* px = x + (((int64_t)b * H + (int64_t)g * rep) * L + t) * D + d;
          float s;
          if (rep == 1) {
            s = px[0];
          } else {
            s = 0.0f;
            for (int h = 0; h < rep; ++h) s = s + px[(int64_t)h * L * D];
            s = rnd(s * inv, dtype);
          }
          out[(((int64_t)b * G + g) * L + t) * D + d] = s;
        }
}

/* a [B,G,L,D] (group-averaged rows) -> out [B,G,nb,P,D]; block <= 64. */
void oracle_proto_pool(const float* a, int B, int G, int L, int D, int block, int P, int dtype, float* out) {
  const int nb = (L + block - 1) / block;
  const int k = P - 1 < block ? P - 1 : block;
  float mean[512];
  float dist[64];
  int taken[64];
  int pick[64];
  for (int b = 0; b < B; ++b)
    for (int g = 0; g < G; ++g)
      for (int i = 0; i < nb; ++i) {
        const float* rows = a + (((int64_t)b * G + g) * L + (int64_t)i * block) * D;
        const int n = L - i * block < block ? L - i * block : block;
        for (int d = 0; d < D; ++d) {
          float s = 0.0f;
          for (int t = 0; t < n; ++t) s = s + rows[(int64_t)t * D + d];
          mean[d] = rnd(rnd(s, dtype) / (float)n, dtype);
        }
        for (int t = 0; t < block; ++t) {
          taken[t] = 0;
          if (t < n) {
            float s = 0.0f;
            for (int d = 0; d < D; ++d) {
              const float diff = rows[(int64_t)t * D + d] - mean[d];
              s = s + diff * diff;
            }
            dist[t] = s;
          } else {
            dist[t] = -INFINITY;
          }
        }
        for (int j = 0; j < k; ++j) {
          int best = -1;
          for (int t = 0; t < block; ++t) {
            if (taken[t]) continue;
            if (best < 0) { best = t; continue; }
            const float v = dist[t], w = dist[best];
            const int better = isnan(v) ? !isnan(w) : (!isnan(w) && v > w);
            if (better) best = t;
          }
          taken[best] = 1;
          pick[j] = best;
        }
        float* o = out + (((int64_t)b * G + g) * nb + i) * (int64_t)P * D;
        for (int pr = 0; pr < P; ++pr)
          for (int d = 0; d < D; ++d) {
            float v = mean[d];
            if (pr >= 1 && pr <= k && pick[pr - 1] < n) v = rows[(int64_t)pick[pr - 1] * D + d];
            o[(int64_t)pr * D + d] = v;
          }
      }
}
