/*
 * CPU oracle for the tree selector -- TEST INFRASTRUCTURE ONLY.
 * Used by tests/ as the checker of the HIP tree kernels.
 *
 * Restates, in the float32 operation order of the HIP kernels:
 *   oracle_tree_merge      one parent level of build_key_tree
 *                          (selector/tree.py:79-145): parent j covers children
 *                          [j*radix, min((j+1)*radix, n)); prototype 0 =
 *                          rnd(rnd(sum_c x_c[0]) / count) (sum from 0.0f in
 *                          child order; the reference sums and divides in the
 *                          model dtype, :93-96); prototypes 1..P-1 = the P-1
 *                          child prototypes farthest from it in float32
 *                          squared L2 (dims in order from 0.0f), farthest
 *                          first, ties to the lower candidate index, NaN
 *                          farthest (:102-109; the reference's distances are
 *                          in the model dtype and its tie order is torch.topk's).
 *   oracle_candidate_scores FlatGate.score_projected_candidates
 *                          (selector/gate.py:129-166): per key prototype c the
 *                          max over query prototypes a (a ascending, strict >)
 *                          of the fmaf chain over the projection dim, then the
 *                          max over c (c ascending, strict >), divided by div.
 *   oracle_tree_traverse   traverse_to_leaf_ids
 *                          (scripts/eval_tree_traversal.py:59-113): from the
 *                          root, each level scores the children of the beam,
 *                          drops children past the last level node or starting
 *                          after the query block, and keeps the
 *                          k = min(beam, candidates, level nodes) best, score
 *                          descending with ties to the lower node, -1 for
 *                          slots without a valid candidate.
 * rnd() rounds to the model dtype, nearest even (dtype 0 bf16, 1 f16, 2 f32).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oracle_round(const float* x, int64_t n, int dtype, float* out);

static float rnd1(float x, int dtype) {
  float y;
  oracle_round(&x, 1, dtype, &y);
  return y;
}

static int ranks_before(float a, int ia, float b, int ib) {
  const int na = isnan(a), nb = isnan(b);
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

/* child [S, n, P, D] -> parent [S, ceil(n/radix), P, D]; floats holding model-dtype values. */
void oracle_tree_merge(const float* child, int S, int n, int P, int D, int radix, int dtype, float* parent) {
  const int m = (n + radix - 1) / radix;
  float* mean = (float*)malloc(sizeof(float) * (size_t)D);
  float* dist = (float*)malloc(sizeof(float) * (size_t)radix * P);
  for (int s = 0; s < S; ++s)
    for (int j = 0; j < m; ++j) {
      const int c0 = j * radix;
      const int cn = n - c0 < radix ? n - c0 : radix;
      const float* x = child + (((size_t)s * n + c0) * P) * D;
      float* out = parent + (((size_t)s * m + j) * P) * D;
      for (int d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int c = 0; c < cn; ++c) acc = acc + x[(size_t)c * P * D + d];
        mean[d] = rnd1(rnd1(acc, dtype) / (float)cn, dtype);
        out[d] = mean[d];
      }
      const int ncand = cn * P;
      for (int i = 0; i < ncand; ++i) {
        float acc = 0.0f;
        for (int d = 0; d < D; ++d) {
          const float df = x[(size_t)i * D + d] - mean[d];
          acc = acc + df * df;
        }
        dist[i] = acc;
      }
      for (int i = 0; i < ncand; ++i) {
        int rank = 0;
        for (int o = 0; o < ncand; ++o) rank += ranks_before(dist[o], o, dist[i], i);
        if (rank < P - 1) memcpy(out + (size_t)(1 + rank) * D, x + (size_t)i * D, sizeof(float) * (size_t)D);
      }
    }
  free(mean);
  free(dist);
}

static float maxsim(const float* q, const float* k, int Pq, int Pk, int pd, float div) {
  float best = 0.0f;
  for (int c = 0; c < Pk; ++c) {
    float mc = 0.0f;
    for (int a = 0; a < Pq; ++a) {
      float acc = 0.0f;
      for (int e = 0; e < pd; ++e) acc = fmaf(q[(size_t)a * pd + e], k[(size_t)c * pd + e], acc);
      if (a == 0 || acc > mc) mc = acc;
    }
    if (c == 0 || mc > best) best = mc;
  }
  return best / div;
}

/* qp [S, qb, Pq, p], kp [S, N, Pk, p], ids [S, qb, C] -> out [S, qb, C]. */
void oracle_candidate_scores(const float* qp, const float* kp, const int32_t* ids, int S, int qb, int N, int C,
                             int Pq, int Pk, int pd, float div, float* out) {
  for (int s = 0; s < S; ++s)
    for (int q = 0; q < qb; ++q)
      for (int i = 0; i < C; ++i) {
        int node = ids[((size_t)s * qb + q) * C + i];
        node = node < 0 ? 0 : (node >= N ? N - 1 : node);
        out[((size_t)s * qb + q) * C + i] =
            maxsim(qp + ((size_t)s * qb + q) * Pq * pd, kp + ((size_t)s * N + node) * Pk * pd, Pq, Pk, pd, div);
      }
}

/* Rows q0 .. q0+nq-1 of every slab; qp [S, nq, Pq, p] holds those rows, out
 * [S, nq, C].  Returns the output width C, or -1 if the tree is too deep. */
int oracle_tree_traverse(const float* qp, const float* kp, int S, int q0, int nq, int kb, int Pq, int Pk, int pd,
                         int radix, int beam, float div, int32_t* out) {
  int count[64], offset[64];
  int64_t span[64];
  int levels = 0, total = 0;
  int64_t cnt = kb, sp = 1;
  while (1) {
    if (levels >= 64) return -1;
    count[levels] = (int)cnt;
    offset[levels] = total;
    span[levels] = sp;
    total += (int)cnt;
    ++levels;
    if (cnt == 1) break;
    cnt = (cnt + radix - 1) / radix;
    sp *= radix;
  }
  int W = 1;
  for (int v = levels - 2; v >= 0; --v) {
    int k = beam < W * radix ? beam : W * radix;
    W = k < count[v] ? k : count[v];
  }
  const int C = W;
  const int maxc = beam * radix > 1 ? beam * radix : 1;
  int* sel = (int*)malloc(sizeof(int) * (size_t)maxc);
  int* nsel = (int*)malloc(sizeof(int) * (size_t)maxc);
  int* cand = (int*)malloc(sizeof(int) * (size_t)maxc);
  int* valid = (int*)malloc(sizeof(int) * (size_t)maxc);
  float* score = (float*)malloc(sizeof(float) * (size_t)maxc);
  for (int s = 0; s < S; ++s)
    for (int r = 0; r < nq; ++r) {
      const int q = q0 + r;
      const float* qrow = qp + ((size_t)s * nq + r) * Pq * pd;
      sel[0] = 0;
      int w = 1;
      for (int v = levels - 2; v >= 0; --v) {
        const int nc = w * radix;
        for (int i = 0; i < nc; ++i) {
          const int par = sel[i / radix];
          cand[i] = par >= 0 ? par * radix + i % radix : -1;
          valid[i] = par >= 0 && cand[i] < count[v] && (int64_t)cand[i] * span[v] <= q;
          score[i] = valid[i] ? maxsim(qrow, kp + ((size_t)s * total + offset[v] + cand[i]) * Pk * pd, Pq, Pk, pd, div)
                              : 0.0f;
        }
        int k = beam < nc ? beam : nc;
        k = k < count[v] ? k : count[v];
        for (int i = 0; i < nc; ++i) {
          int rank = 0;
          for (int o = 0; o < nc; ++o) {
            if (o == i) continue;
            int before;
            if (valid[o] != valid[i]) before = valid[o];
            else if (!valid[o]) before = o < i;
            else before = ranks_before(score[o], cand[o], score[i], cand[i]);
            rank += before;
          }
          if (rank < k) nsel[rank] = valid[i] ? cand[i] : -1;
        }
        memcpy(sel, nsel, sizeof(int) * (size_t)k);
        w = k;
      }
      for (int i = 0; i < C; ++i) out[((size_t)s * nq + r) * C + i] = sel[i];
    }
  free(sel);
  free(nsel);
  free(cand);
  free(valid);
  free(score);
  return C;
}
