/*
 * CPU oracle for the selector front end -- TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the shipped package links this file: tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it (oracle/_build/liboracle_selector.so)
 * as the checker of the HIP selector kernels.
 *
 * Selected block indices must match the GPU bit for bit, so every floating
 * point result here is produced by the same sequence of IEEE single-precision
 * operations the kernels execute (build with -ffp-contract=off; fused
 * multiply-adds only where fmaf() is written):
 *
 *   pool  : per token, the G query heads of a KV group are summed left to right
 *           (h = 0..G-1); token t of a 64-token block goes to lane t % L (L =
 *           the largest power of two <= min(64, 256 / (D/8)) lanes per dim, so
 *           that the lanes cover the block and the halving tree every lane;
 *           tests/test_oracle_selector.py also checks the means against plain
 *           float64 block means at such D), each lane folds its tokens in
 *           increasing order (starting from the first token's value), lanes are
 *           combined by a halving tree (lane i += lane i + s for s = L/2, L/4,
 *           .., 1), and the block sum is divided (IEEE division) by
 *           G * (real tokens of the block).  Missing tokens of a ragged last
 *           block contribute +0.0f to the sums and nothing to the max.  K
 *           blocks get the same mean (G = 1) plus an exact per-dim max.
 *           Follows teacher/chunked_extract.py:75-80 (_group_avg_tokens) and
 *           :27-72 prototype 0 (_proto_pool_seq block mean) in float32, and
 *           adds the per-dim max summary the cfg3 workload defines.
 *   project: out[n][j] = fmaf chain over d = 0..D-1 of x[n][d] * W[d][j],
 *           starting from 0 (selector/gate.py:120-127, x @ W with W [d, p]).
 *   scores: score[i][j] = max over prototype pairs (a, c), in order a-major,
 *           of the fmaf chain over the projection dim, divided by `div`
 *           (= (float)sqrt(p)); with `causal`, j > i is -inf (selector/gate.py:
 *           29-101, selector/recall.py:26-35 causal mask).
 *   topk  : per row the k causal entries with the largest score, ties to the
 *           lower block index (stable descending argsort,
 *           selector/baselines.py:59-62), returned ascending with -1 padding
 *           (the selected_blocks row layout, interfaces/selected_blocks_spec.md).
 *           Implemented as a comparison sort, independent of the GPU's radix
 *           select.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static const int kBlock = 64;

/* q: float32 [B, Hq, T, D] contiguous (bf16 values widened exactly), may be NULL.
 * k: float32 [B, Hkv, T, D] contiguous, may be NULL.
 * q_mean: [B, Hkv, nb, D];  k_sum: [B, Hkv, nb, 2, D] (mean, max). */
void oracle_block_pool(const float* q, const float* k, int B, int Hq, int Hkv, int T, int D,
                       float* q_mean, float* k_sum) {
  const int nb = (T + kBlock - 1) / kBlock;
  const int G = Hq / Hkv;
  const int dch = D / 8;
  int L = kBlock; /* token lanes per dim chunk: a power of two, L * dch <= 256 */
  while (L > 1 && L * dch > 256) L /= 2;
  const int per = kBlock / L;         /* tokens folded by one lane */
  float lanes[64];
  for (int b = 0; b < B; ++b)
    for (int g = 0; g < Hkv; ++g)
      for (int blk = 0; blk < nb; ++blk) {
        const int t0 = blk * kBlock;
        int n = T - t0;
        if (n > kBlock) n = kBlock;
        for (int d = 0; d < D; ++d) {
          if (q) {
            for (int l = 0; l < L; ++l) {
              float acc = 0.f;
              for (int i = 0; i < per; ++i) {
                const int t = t0 + l + i * L;
                float s = 0.f;
                if (t < T) {
                  const float* base = q + (((size_t)b * Hq + (size_t)g * G) * T + t) * D + d;
                  s = base[0];
                  for (int h = 1; h < G; ++h) s = s + base[(size_t)h * T * D];
                }
                acc = (i == 0) ? s : acc + s;
              }
              lanes[l] = acc;
            }
            for (int st = L / 2; st >= 1; st /= 2)
              for (int l = 0; l < st; ++l) lanes[l] = lanes[l] + lanes[l + st];
            q_mean[(((size_t)b * Hkv + g) * nb + blk) * D + d] = lanes[0] / (float)(G * n);
          }
          if (k) {
            float mx = -INFINITY;
            for (int l = 0; l < L; ++l) {
              float acc = 0.f;
              for (int i = 0; i < per; ++i) {
                const int t = t0 + l + i * L;
                float s = 0.f;
                if (t < T) {
                  s = k[(((size_t)b * Hkv + g) * T + t) * D + d];
                  if (s > mx || (s == mx && signbit(mx) && !signbit(s))) mx = s;
                }
                acc = (i == 0) ? s : acc + s;
              }
              lanes[l] = acc;
            }
            for (int st = L / 2; st >= 1; st /= 2)
              for (int l = 0; l < st; ++l) lanes[l] = lanes[l] + lanes[l + st];
            float* out = k_sum + ((((size_t)b * Hkv + g) * nb + blk) * 2) * D + d;
            out[0] = lanes[0] / (float)n;
            out[D] = mx;
          }
        }
      }
}

/* out[n][j] = sum_d x[n][d] * W[d][j] as a sequential fmaf chain. */
void oracle_project(const float* x, const float* W, int N, int D, int P, float* out) {
  for (int n = 0; n < N; ++n)
    for (int j = 0; j < P; ++j) {
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc = fmaf(x[(size_t)n * D + d], W[(size_t)d * P + j], acc);
      out[(size_t)n * P + j] = acc;
    }
}

/* qp: [BG, Qb, Pq, P], kp: [BG, Kb, Pk, P], scores: [BG, Qb, Kb]. */
void oracle_scores(const float* qp, const float* kp, int BG, int Qb, int Kb, int Pq, int Pk, int P,
                   float div, int causal, float* scores) {
  for (int bg = 0; bg < BG; ++bg)
    for (int i = 0; i < Qb; ++i)
      for (int j = 0; j < Kb; ++j) {
        float best = -INFINITY;
        if (!causal || j <= i) {
          for (int a = 0; a < Pq; ++a)
            for (int c = 0; c < Pk; ++c) {
              const float* x = qp + (((size_t)bg * Qb + i) * Pq + a) * P;
              const float* y = kp + (((size_t)bg * Kb + j) * Pk + c) * P;
              float acc = 0.f;
              for (int e = 0; e < P; ++e) acc = fmaf(x[e], y[e], acc);
              if (a == 0 && c == 0) best = acc;
              else if (acc > best) best = acc;
            }
          best = best / div;
        }
        scores[((size_t)bg * Qb + i) * Kb + j] = best;
      }
}

typedef struct {
  float s;
  int i;
} Entry;

static int by_score_desc(const void* a, const void* b) {
  const Entry* x = (const Entry*)a;
  const Entry* y = (const Entry*)b;
  if (x->s > y->s) return -1;
  if (x->s < y->s) return 1;
  return x->i - y->i; /* ties: lower index first */
}

static int by_int(const void* a, const void* b) { return *(const int*)a - *(const int*)b; }

/* scores: [R, Qb, Kb] (row i of each slab considers j <= i); out: [R, Qb, k]. */
void oracle_topk(const float* scores, int R, int Qb, int Kb, int k, int32_t* out) {
  Entry* e = (Entry*)malloc(sizeof(Entry) * (size_t)Kb);
  int* sel = (int*)malloc(sizeof(int) * (size_t)(k > 0 ? k : 1));
  for (int r = 0; r < R; ++r)
    for (int i = 0; i < Qb; ++i) {
      int n = i + 1 < Kb ? i + 1 : Kb;
      const float* row = scores + ((size_t)r * Qb + i) * Kb;
      for (int j = 0; j < n; ++j) {
        e[j].s = row[j];
        e[j].i = j;
      }
      qsort(e, (size_t)n, sizeof(Entry), by_score_desc);
      const int m = n < k ? n : k;
      for (int t = 0; t < m; ++t) sel[t] = e[t].i;
      qsort(sel, (size_t)m, sizeof(int), by_int);
      int32_t* o = out + ((size_t)r * Qb + i) * k;
      for (int t = 0; t < k; ++t) o[t] = t < m ? sel[t] : -1;
    }
  free(e);
  free(sel);
}
