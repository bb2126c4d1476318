// Tree selector on gfx950: the key-axis prototype tree and its top-down beam
// traversal, the deployed route producer.
//
//   tree_merge_kernel     one parent level of build_key_tree
//   tree_merge_top_kernel the narrow levels near the root, in one launch
//                         (selector/tree.py:79-145, _merge_level_prototypes)
//   tree_traverse_kernel  traverse_to_leaf_ids
//                         (scripts/eval_tree_traversal.py:59-113)
//   candidate_scores_kernel FlatGate.score_projected_candidates
//                         (selector/gate.py:129-166)
//
// Every float is produced by a fixed IEEE single-precision operation
// sequence (this file is built without contraction, with IEEE division and
// denormals), so node choices are reproducible bit for bit by a CPU
// restatement:
//   merge:  prototype 0 of parent j = rnd(rnd(sum_c x_c) / n) over its n
//           valid children's prototype 0 (sum from 0.0f, children in order;
//           rnd = round to the model dtype, as the reference's model-dtype
//           sum and division do); prototypes 1..P-1 = the P-1 child
//           prototypes farthest from it in float32 squared L2 (dims summed in
//           order from 0.0f), farthest first, ties to the lower candidate
//           index (child-major, prototype-minor), NaN farthest.
//   score:  for key prototype c, the max over query prototypes a (a
//           ascending, strict >) of the fmaf chain over the projection dim
//           from 0.0f; then the max over c (c ascending, strict >); divided
//           by `div` (= fl(sqrt(p))).
//   beam:   per level the k = min(beam, candidates, level nodes) valid
//           candidates with the largest score, ties to the lower node index,
//           score-descending; missing slots are -1 (the reference ranks
//           invalid candidates at finfo.min after every valid one).
#include "common.h"

namespace spruce {

namespace {

constexpr int kMaxLevels = 40;

__device__ __forceinline__ float model_round(float x, int dtype) {
  if (dtype == SPRUCE_DTYPE_BF16) return (float)(__bf16)x;
  if (dtype == SPRUCE_DTYPE_F16) return (float)(_Float16)x;
  return x;
}

__device__ __forceinline__ float load_elem(const void* base, int64_t i, int dtype) {
  if (dtype == SPRUCE_DTYPE_F32) return static_cast<const float*>(base)[i];
  const uint16_t b = static_cast<const uint16_t*>(base)[i];
  return dtype == SPRUCE_DTYPE_F16 ? unpack1<true>(b) : unpack1<false>(b);
}

__device__ __forceinline__ void store_elem(void* base, int64_t i, float v, int dtype) {
  if (dtype == SPRUCE_DTYPE_F32) {
    static_cast<float*>(base)[i] = v;
  } else if (dtype == SPRUCE_DTYPE_F16) {
    static_cast<_Float16*>(base)[i] = (_Float16)v;
  } else {
    static_cast<__bf16*>(base)[i] = (__bf16)v;
  }
}

// Order-preserving 32-bit image of a score: larger score -> larger image,
// every NaN the largest, -0 and +0 equal (the order of ranks_before).
__device__ __forceinline__ uint32_t score_order(float x) {
  if (x != x) return 0xffffffffu;
  if (x == 0.f) return 0x80000000u;
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// a ranks before b: larger value first, NaN largest, ties to the lower index.
__device__ __forceinline__ bool ranks_before(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

struct MergeParams {
  const void* child;  // [S, n, P, D]
  void* parent;       // [S, m, P, D]
  int64_t S;
  int n, m, P, D, radix, dtype;
  int vec;            // D % 8 == 0 and child 16-byte aligned: 8-element loads
};

// Orders a wavefront's LDS stores before its later LDS loads.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Parent j of slab s, merged by one wavefront (lane 0..63) in its own LDS
// region sh of merge_lds_floats(p) floats.
__device__ __forceinline__ void merge_parent(const MergeParams& p, int64_t s, int j, int lane, float* sh) {
  const int c0 = j * p.radix;
  const int cn = p.n - c0 < p.radix ? p.n - c0 : p.radix;  // valid children
  const int ncand = cn * p.P;
  const int D = p.D;
  // Rows padded to D + 4 floats: 16-byte aligned and spread over the banks.
  const int FS = D + 4;
  float* feat = sh;                   // [ncand, FS]
  float* mean = feat + ncand * FS;    // [D]
  const int64_t cbase = ((s * p.n + c0) * p.P) * (int64_t)D;
  if (p.vec) {
    // 8 elements per load, up to 4 loads per lane in flight before the LDS
    // stores (one round trip per 2048 elements).
    const int nv = ncand * D / 8;
    for (int v0 = 0; v0 < nv; v0 += 256) {
      float t[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int vi = v0 + 64 * u + lane;
        if (vi < nv) load8f(p.child, cbase + 8 * (int64_t)vi, p.dtype, t[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int vi = v0 + 64 * u + lane;
        if (vi < nv) {
          const int row = (8 * vi) / D, col = 8 * vi - row * D;
#pragma unroll
          for (int j = 0; j < 8; ++j) feat[row * FS + col + j] = t[u][j];
        }
      }
    }
  } else {
    for (int i = lane; i < ncand * D; i += 64) feat[(i / D) * FS + i % D] = load_elem(p.child, cbase + i, p.dtype);
  }
  wave_sync();
  for (int d = lane; d < D; d += 64) {
    float acc = 0.f;
    for (int c = 0; c < cn; ++c) acc = acc + feat[(c * p.P) * FS + d];
    mean[d] = model_round(model_round(acc, p.dtype) / (float)cn, p.dtype);
  }
  wave_sync();
  // Distances in registers: lane i holds candidate i's (dims in order).
  float dist = 0.f;
  if (lane < ncand) {
    float acc = 0.f;
    const float* x = feat + lane * FS;
    if ((D & 3) == 0) {
#pragma unroll 8
      for (int d = 0; d < D; d += 4) {
        const float4 xv = *reinterpret_cast<const float4*>(x + d);
        const float4 mv = *reinterpret_cast<const float4*>(mean + d);
        float df = xv.x - mv.x;
        acc = acc + df * df;
        df = xv.y - mv.y;
        acc = acc + df * df;
        df = xv.z - mv.z;
        acc = acc + df * df;
        df = xv.w - mv.w;
        acc = acc + df * df;
      }
    } else {
      for (int d = 0; d < D; ++d) {
        const float df = x[d] - mean[d];
        acc = acc + df * df;
      }
    }
    dist = acc;
  }
  const int64_t pbase = (s * p.m + j) * (int64_t)p.P * D;
  for (int d = lane; d < D; d += 64) store_elem(p.parent, pbase + d, mean[d], p.dtype);
  if (p.P > 1) {
    int rank = 64;
    if (lane < ncand) {
      rank = 0;
      for (int o = 0; o < ncand; ++o) {
        const float od = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dist), o));
        rank += ranks_before(od, o, dist, lane) ? 1 : 0;
      }
    }
    // Slot 1 + r takes the candidate of rank r (ranks are a permutation of
    // 0..ncand-1, and ncand >= P > P - 1).
    for (int r = 0; r < p.P - 1; ++r) {
      const int src = __builtin_ctzll(__ballot(rank == r));
      for (int d = lane; d < D; d += 64)
        store_elem(p.parent, pbase + (int64_t)(1 + r) * D + d, feat[src * FS + d], p.dtype);
    }
  }
}

// One wavefront per (slab, parent node).
__global__ __launch_bounds__(64) void tree_merge_kernel(const MergeParams p) {
  extern __shared__ float sh[];
  const int64_t g = blockIdx.x;
  const int64_t s = g / p.m;
  const int j = (int)(g - s * p.m);
  if (s >= p.S) return;
  merge_parent(p, s, j, threadIdx.x, sh);
}

// The narrow levels near the root in one launch, where a launch per level
// costs more than its work: one workgroup of up to kTopWaves wavefronts per
// slab; wavefront w merges parents w, w + (wavefronts), ... of a level with
// merge_parent, and a workgroup barrier separates the levels (a level's
// parents are the next level's children, read back after the barrier from
// the same workgroup's stores).
constexpr int kTopWaves = 16, kMergeTopMax = 32;
struct MergeTopParams {
  MergeParams p;                   // S, P, D, radix, dtype
  int levels;                      // parent levels to form
  int n[kMergeTopMax + 1];         // node count of each level; n[0] = the input's
  void* lvl[kMergeTopMax + 1];     // lvl[0] = input, lvl[v] = parent level v
  int vec[kMergeTopMax];           // the vec flag of level v as a child
  int wave_lds;                    // LDS floats per wavefront
};

__global__ __launch_bounds__(64 * kTopWaves) void tree_merge_top_kernel(const MergeTopParams t) {
  extern __shared__ float sh[];
  const int64_t s = blockIdx.x;
  const int nw = (int)(blockDim.x >> 6);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  float* mine = sh + wave * t.wave_lds;
  for (int v = 0; v < t.levels; ++v) {
    MergeParams p = t.p;
    p.child = t.lvl[v];
    p.parent = t.lvl[v + 1];
    p.n = t.n[v];
    p.m = t.n[v + 1];
    p.vec = t.vec[v];
    for (int j = wave; j < p.m; j += nw) merge_parent(p, s, j, lane, mine);
    __syncthreads();
  }
}

struct ScoreParams2 {
  const float* qp;  // [S, qb, Pq, p]
  const float* kp;  // [S, N, Pk, p] (rows) or [S, N, p/4, Pk, 4] (interleaved)
  int64_t S;
  int qb, N, Pq, Pk, pd;
  float div;
  int cstride;      // floats from a node's prototype c to c + 1: p (rows) or 4
  int gs;           // floats from a prototype's 4-float group to the next: 4 or 4 * Pk
};

// Offset of prototype c of node `node` (counted from the table's start).
__device__ __forceinline__ int64_t kvec(const ScoreParams2& sc, int64_t node, int c) {
  return node * sc.Pk * (int64_t)sc.pd + (int64_t)c * sc.cstride;
}

// Max over query prototypes of q_a . k (fmaf chains over the projection dim,
// all a at once; each chain runs e = 0..p-1 in order).  qrow in LDS.
__device__ __forceinline__ float maxsim_one(const float* qrow, const float* krow, int Pq, int pd, int gs) {
  float acc[16];
#pragma unroll
  for (int a = 0; a < 16; ++a) acc[a] = 0.f;
  // The key vector (4-float groups gs floats apart) streams from L2 one
  // group ahead of its use.
  float4 knext = *reinterpret_cast<const float4*>(krow);
  for (int e = 0; e < pd; e += 4) {
    const float4 k4 = knext;
    if (e + 4 < pd) knext = *reinterpret_cast<const float4*>(krow + (int64_t)(e / 4 + 1) * gs);
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      if (a < Pq) {
        const float4 q4 = *reinterpret_cast<const float4*>(qrow + a * pd + e);
        float t = acc[a];
        t = fmaf(q4.x, k4.x, t);
        t = fmaf(q4.y, k4.y, t);
        t = fmaf(q4.z, k4.z, t);
        t = fmaf(q4.w, k4.w, t);
        acc[a] = t;
      }
    }
  }
  float best = acc[0];
#pragma unroll
  for (int a = 1; a < 16; ++a)
    if (a < Pq && acc[a] > best) best = acc[a];
  return best;
}

// NP (candidate, key prototype) pairs per lane against a compile-time number
// of query prototypes: every query float4 read from LDS feeds all NP pairs,
// and each chain is the same fmaf sequence as maxsim_one (e ascending), so
// the results are identical.  The key vectors stream in pieces of CW float4
// (loads back to back): lanes read different vectors, and taking a line in a
// few pieces close together keeps it in L1 between them, where one float4
// per step was refetched from L2 for every 16 bytes (measured 1.85 -> 1.0-1.1
// ms at the cfg5 grid).  Two register sets take the pieces in turn, the next
// piece loading while the other is used, so no piece is copied between
// registers (the loads are unconditional: the last one re-reads piece 0,
// in bounds and unused).  Requires pd % (8 * CW) == 0; PD > 0 fixes pd at
// compile time, so the query reads take immediate LDS offsets, and GS > 0
// the key group stride (4: rows layout; 4 * Pk: interleaved, where the Pk
// prototypes of a node that neighbouring lanes hold share each 16 * Pk-byte
// group, so a load touches one line per node instead of one per lane).
template <int NP, int CW, int GS>
__device__ __forceinline__ void load_piece(const float* const (&kv)[NP], int e0, int gs_rt, float4 (&k)[NP][CW]) {
  const int gs = GS > 0 ? GS : gs_rt;
#pragma unroll
  for (int n = 0; n < NP; ++n)
#pragma unroll
    for (int j = 0; j < CW; ++j)
      k[n][j] = *reinterpret_cast<const float4*>(kv[n] + (int64_t)(e0 / 4 + j) * gs);
}

template <int PQ, int NP, int CW, int PD>
__device__ __forceinline__ void fma_piece(const float* qrow, int pd_rt, int e0, const float4 (&k)[NP][CW],
                                          float (&acc)[NP][PQ]) {
  const int pd = PD > 0 ? PD : pd_rt;
#pragma unroll
  for (int j = 0; j < CW; ++j) {
    const int e = e0 + 4 * j;
#pragma unroll
    for (int a = 0; a < PQ; ++a) {
      const float4 q4 = *reinterpret_cast<const float4*>(qrow + a * pd + e);
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        float t = acc[n][a];
        t = fmaf(q4.x, k[n][j].x, t);
        t = fmaf(q4.y, k[n][j].y, t);
        t = fmaf(q4.z, k[n][j].z, t);
        t = fmaf(q4.w, k[n][j].w, t);
        acc[n][a] = t;
      }
    }
  }
}

template <int PQ, int NP, int CW, int PD, int GS>
__device__ __forceinline__ void maxsim_multi(const float* qrow, const float* const (&kv)[NP], int pd_rt, int gs,
                                             float (&res)[NP]) {
  const int pd = PD > 0 ? PD : pd_rt;
  float acc[NP][PQ];
#pragma unroll
  for (int n = 0; n < NP; ++n)
#pragma unroll
    for (int a = 0; a < PQ; ++a) acc[n][a] = 0.f;
  constexpr int kStep = 4 * CW;
  float4 ka[NP][CW], kb[NP][CW];
  load_piece<NP, CW, GS>(kv, 0, gs, ka);
  for (int e0 = 0; e0 < pd; e0 += 2 * kStep) {
    load_piece<NP, CW, GS>(kv, e0 + kStep, gs, kb);
    fma_piece<PQ, NP, CW, PD>(qrow, pd, e0, ka, acc);
    load_piece<NP, CW, GS>(kv, e0 + 2 * kStep < pd ? e0 + 2 * kStep : 0, gs, ka);
    fma_piece<PQ, NP, CW, PD>(qrow, pd, e0 + kStep, kb, acc);
  }
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    float x = acc[n][0];
#pragma unroll
    for (int a = 1; a < PQ; ++a)
      if (acc[n][a] > x) x = acc[n][a];
    res[n] = x;
  }
}

// Two pairs per lane in 64-byte pieces.  Measured at the cfg5 grid against
// 1.0-1.06 ms: four pairs in 64-byte pieces 1.68 ms (289 registers), four in
// 32-byte pieces 1.10 ms, four or eight in 16-byte pieces 1.77-2.03 ms.
constexpr int kTravNP = 2, kTravCW = 4;

struct TraverseParams {
  ScoreParams2 sc;
  int kb, radix, beam, levels, C;
  int count[kMaxLevels];
  int offset[kMaxLevels];
  int64_t span[kMaxLevels];  // leaves per node at each level (radix^v)
  int32_t* out;              // [S, qb, C]
};

// Scores pairs pr + 64 n (n < NP) of one level into pm.  An invalid or
// missing pair reads the level's first node (always in range) and its result
// is dropped.
template <int PQ, int NP, int PD, int GS>
__device__ __forceinline__ void score_pairs(const ScoreParams2& sc, const float* qrow, const float* kl,
                                            const int* cand, const int* valid, int npairs, int lane,
                                            float* pm) {
  for (int pr = lane; pr < npairs; pr += 64 * NP) {
    int idx[NP], cc[NP];
    bool ok[NP];
    const float* kv[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const int pn = pr + 64 * n;
      idx[n] = pn < npairs ? pn / sc.Pk : 0;
      cc[n] = pn < npairs ? pn - idx[n] * sc.Pk : 0;
      ok[n] = pn < npairs && valid[idx[n]] != 0;
      kv[n] = kl + (ok[n] ? kvec(sc, cand[idx[n]], cc[n]) : 0);
    }
    float m[NP];
    maxsim_multi<PQ, NP, kTravCW, PD, GS>(qrow, kv, sc.pd, sc.gs, m);
#pragma unroll
    for (int n = 0; n < NP; ++n)
      if (pr + 64 * n < npairs) pm[idx[n] * sc.Pk + cc[n]] = ok[n] ? m[n] : 0.f;
  }
}

// One wavefront per (slab, query block) row.  PQ > 0: that many query
// prototypes, two pairs per lane per step (one on levels of at most 64
// pairs); PQ == 0: any count, one pair.
template <int PQ, int PD = 0, int GS = 0>
__global__ __launch_bounds__(64) void tree_traverse_kernel(const TraverseParams p) {
  extern __shared__ float sh[];
  const ScoreParams2& sc = p.sc;
  const int64_t row = blockIdx.x;
  const int64_t s = row / sc.qb;
  const int q = (int)(row - s * sc.qb);
  if (s >= sc.S) return;
  const int lane = threadIdx.x;
  float* qrow = sh;                          // [Pq, p]
  float* pm = qrow + sc.Pq * sc.pd;          // [64, Pk] per-(candidate, key prototype) max
  int* cand = reinterpret_cast<int*>(pm + 64 * sc.Pk);   // [64]
  int* valid = cand + 64;                    // [64]
  int* sel = valid + 64;                     // [64] current beam (node index within level)
  const float* qsrc = sc.qp + (s * sc.qb + q) * (int64_t)sc.Pq * sc.pd;
  for (int i = lane; i < sc.Pq * sc.pd; i += 64) qrow[i] = qsrc[i];
  if (lane == 0) sel[0] = 0;  // the root
  int W = 1;
  __syncthreads();
  for (int v = p.levels - 2; v >= 0; --v) {
    const int ncand = W * p.radix;
    if (lane < ncand) {
      const int par = sel[lane / p.radix];
      const int c = par >= 0 ? par * p.radix + lane % p.radix : -1;
      const bool ok = par >= 0 && c < p.count[v] && (int64_t)c * p.span[v] <= q;
      cand[lane] = c;
      valid[lane] = ok ? 1 : 0;
    }
    __syncthreads();
    const float* kl = sc.kp + (s * sc.N + p.offset[v]) * (int64_t)sc.Pk * sc.pd;
    const int npairs = ncand * sc.Pk;
    if (PQ > 0 && sc.pd % (8 * kTravCW) == 0) {
      // A level with at most 64 pairs (the tree's top levels) takes one pair
      // per lane: with two, half of every lane's chains would be dropped.
      if (npairs <= 64)
        score_pairs<PQ == 0 ? 1 : PQ, 1, PD, GS>(sc, qrow, kl, cand, valid, npairs, lane, pm);
      else
        score_pairs<PQ == 0 ? 1 : PQ, kTravNP, PD, GS>(sc, qrow, kl, cand, valid, npairs, lane, pm);
    } else {
      for (int pr = lane; pr < npairs; pr += 64) {
        const int i = pr / sc.Pk, c = pr - (pr / sc.Pk) * sc.Pk;
        float m = 0.f;
        if (valid[i]) m = maxsim_one(qrow, kl + kvec(sc, cand[i], c), sc.Pq, sc.pd, sc.gs);
        pm[i * sc.Pk + c] = m;
      }
    }
    __syncthreads();
    // Each candidate's place in the order (valid first; then score
    // descending, NaN first, equal scores to the lower node; invalid ones by
    // lane) as one distinct 64-bit key, larger = earlier, so a rank is a
    // count of larger keys: one 64-bit compare per other candidate.
    uint64_t key = 0;
    if (lane < ncand) {
      float best = pm[lane * sc.Pk];
      for (int c = 1; c < sc.Pk; ++c)
        if (pm[lane * sc.Pk + c] > best) best = pm[lane * sc.Pk + c];
      key = valid[lane] ? (1ull << 63) | ((uint64_t)score_order(best / sc.div) << 31) |
                              (uint64_t)(0x7fffffff - cand[lane])
                        : (uint64_t)(63 - lane);
    }
    int k = p.beam < ncand ? p.beam : ncand;
    k = k < p.count[v] ? k : p.count[v];
    int rank = 0;
    for (int o = 0; o < ncand; ++o) {
      const uint64_t ko = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key >> 32), o) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, o);
      rank += ko > key ? 1 : 0;
    }
    if (lane < ncand && rank < k) sel[rank] = valid[lane] ? cand[lane] : -1;
    W = k;
    __syncthreads();
  }
  int32_t* o = p.out + row * (int64_t)p.C;
  for (int i = lane; i < p.C; i += 64) o[i] = i < W ? sel[i] : -1;
}

struct CandParams {
  ScoreParams2 sc;
  const int32_t* ids;  // [S, qb, C]
  int C;
  float* out;          // [S, qb, C]
};

// One wavefront per (slab, query block) row; lanes over (candidate, key prototype).
__global__ __launch_bounds__(64) void candidate_scores_kernel(const CandParams p) {
  extern __shared__ float sh[];
  const ScoreParams2& sc = p.sc;
  const int64_t row = blockIdx.x;
  const int64_t s = row / sc.qb;
  if (s >= sc.S) return;
  const int lane = threadIdx.x;
  float* qrow = sh;
  float* pm = qrow + sc.Pq * sc.pd;  // [64, Pk]
  const float* qsrc = sc.qp + row * (int64_t)sc.Pq * sc.pd;
  for (int i = lane; i < sc.Pq * sc.pd; i += 64) qrow[i] = qsrc[i];
  __syncthreads();
  const int32_t* idr = p.ids + row * (int64_t)p.C;
  for (int c0 = 0; c0 < p.C; c0 += 64) {
    const int nc = p.C - c0 < 64 ? p.C - c0 : 64;
    for (int pr = lane; pr < nc * sc.Pk; pr += 64) {
      const int i = pr / sc.Pk, c = pr - (pr / sc.Pk) * sc.Pk;
      int node = idr[c0 + i];
      node = node < 0 ? 0 : (node >= sc.N ? sc.N - 1 : node);  // clamped like the reference
      pm[i * sc.Pk + c] = maxsim_one(qrow, sc.kp + kvec(sc, s * sc.N + node, c), sc.Pq, sc.pd, sc.gs);
    }
    __syncthreads();
    if (lane < nc) {
      float best = pm[lane * sc.Pk];
      for (int c = 1; c < sc.Pk; ++c)
        if (pm[lane * sc.Pk + c] > best) best = pm[lane * sc.Pk + c];
      p.out[row * (int64_t)p.C + c0 + lane] = best / sc.div;
    }
    __syncthreads();
  }
}

int check_score_args(const float* qp, const float* kp, int64_t S, int64_t qb, int64_t N, int64_t Pq, int64_t Pk,
                     int64_t pd, float div) {
  SPRUCE_REQUIRE(qp && kp, "projected query and key pointers must be non-null");
  SPRUCE_REQUIRE(S >= 1 && qb >= 1 && N >= 1, "S, qb and N must be positive");
  SPRUCE_REQUIRE(Pq >= 1 && Pq <= 16, "query prototypes must be in [1, 16], got %lld", (long long)Pq);
  SPRUCE_REQUIRE(Pk >= 1 && Pk <= 64, "key prototypes must be in [1, 64], got %lld", (long long)Pk);
  SPRUCE_REQUIRE(pd >= 4 && pd % 4 == 0 && Pq * pd <= 8192, "projection dim must be a multiple of 4 with Pq*p <= 8192");
  SPRUCE_REQUIRE(((uintptr_t)qp % 16) == 0 && ((uintptr_t)kp % 16) == 0, "projections must be 16-byte aligned");
  SPRUCE_REQUIRE(div > 0.f, "div must be positive");
  SPRUCE_REQUIRE(S * qb < ((int64_t)1 << 31), "too many rows");
  return SPRUCE_OK;
}

}  // namespace
}  // namespace spruce

using namespace spruce;

extern "C" int spruce_tree_merge_level(const void* child, int64_t S, int64_t n, int64_t P, int64_t D, int64_t radix,
                                       int dtype, void* parent, void* stream) {
  SPRUCE_REQUIRE(child && parent, "child and parent must be non-null device pointers");
  SPRUCE_REQUIRE(S >= 1 && n >= 1 && P >= 1 && D >= 1, "S, n, P and D must be positive");
  SPRUCE_REQUIRE(radix >= 2, "radix must be >= 2, got %lld", (long long)radix);
  // Each factor is bounded before the product is formed, so it cannot overflow.
  SPRUCE_REQUIRE(radix <= 64 && P <= 64 && radix * P <= 64, "radix * P must be <= 64, got radix %lld, P %lld",
                 (long long)radix, (long long)P);
  SPRUCE_REQUIRE(D <= 256, "feature dim must be <= 256, got %lld", (long long)D);
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  MergeParams p{};
  p.child = child;
  p.parent = parent;
  p.S = S;
  p.n = (int)n;
  p.m = (int)((n + radix - 1) / radix);
  p.P = (int)P;
  p.D = (int)D;
  p.radix = (int)radix;
  p.dtype = dtype;
  p.vec = (D % 8 == 0 && ((uintptr_t)child % 16) == 0) ? 1 : 0;
  SPRUCE_REQUIRE(S * p.m < ((int64_t)1 << 31), "too many parent nodes");
  const size_t lds = ((size_t)radix * P * (D + 4) + D) * sizeof(float);
  SPRUCE_REQUIRE(lds <= 65536, "radix * P * D too large for one workgroup's LDS (%zu bytes)", lds);
  hipLaunchKernelGGL(tree_merge_kernel, dim3((unsigned)(S * p.m)), dim3(64), lds, (hipStream_t)stream, p);
  return check_launch("tree_merge_kernel");
}

extern "C" int spruce_tree_merge_levels(const void* child, int64_t S, int64_t n, int64_t P, int64_t D,
                                        int64_t radix, int dtype, void* const* parents, int64_t levels,
                                        void* stream) {
  SPRUCE_REQUIRE(child && parents, "child and parents must be non-null");
  SPRUCE_REQUIRE(levels >= 1 && levels <= kMergeTopMax, "levels must be in [1, %d], got %lld", kMergeTopMax,
                 (long long)levels);
  SPRUCE_REQUIRE(S >= 1 && S < ((int64_t)1 << 31) && n >= 1 && n < ((int64_t)1 << 31),
                 "S and n must be in [1, 2^31)");
  SPRUCE_REQUIRE(radix >= 2, "radix must be >= 2, got %lld", (long long)radix);
  SPRUCE_REQUIRE(P >= 1 && D >= 1, "P and D must be positive");
  // The per-level limits of spruce_tree_merge_level, checked before any product below is formed.
  SPRUCE_REQUIRE(radix <= 64 && P <= 64 && radix * P <= 64, "radix * P must be <= 64, got radix %lld, P %lld",
                 (long long)radix, (long long)P);
  SPRUCE_REQUIRE(D <= 256, "feature dim must be <= 256, got %lld", (long long)D);
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  for (int v = 0; v < levels; ++v) SPRUCE_REQUIRE(parents[v], "parent level %d is a null pointer", v);
  const int64_t wave_lds = radix * P * (D + 4) + D;
  int64_t waves = wave_lds > 0 ? 65536 / (wave_lds * (int64_t)sizeof(float)) : 0;
  waves = waves > kTopWaves ? kTopWaves : waves;
  int64_t cur_n = n;
  const void* cur = child;
  for (int v = 0; v < levels; ++v) {
    const int64_t m = (cur_n + radix - 1) / radix;
    if (m <= waves) {
      // Every remaining level has at most one parent per wavefront.
      MergeTopParams t{};
      t.p.S = S;
      t.p.P = (int)P;
      t.p.D = (int)D;
      t.p.radix = (int)radix;
      t.p.dtype = dtype;
      t.levels = (int)(levels - v);
      t.n[0] = (int)cur_n;
      t.lvl[0] = const_cast<void*>(cur);
      for (int u = 0; u < t.levels; ++u) {
        t.n[u + 1] = (t.n[u] + (int)radix - 1) / (int)radix;
        t.lvl[u + 1] = parents[v + u];
        t.vec[u] = (D % 8 == 0 && ((uintptr_t)t.lvl[u] % 16) == 0) ? 1 : 0;
      }
      t.wave_lds = (int)wave_lds;
      const size_t lds = (size_t)waves * wave_lds * sizeof(float);
      hipLaunchKernelGGL(tree_merge_top_kernel, dim3((unsigned)S), dim3((unsigned)(64 * waves)), lds,
                         (hipStream_t)stream, t);
      return check_launch("tree_merge_top_kernel");
    }
    // Wide level: one wavefront per parent (checks every argument).
    const int rc = spruce_tree_merge_level(cur, S, cur_n, P, D, radix, dtype, parents[v], stream);
    if (rc != 0) return rc;
    cur = parents[v];
    cur_n = m;
  }
  return 0;
}

extern "C" int spruce_tree_traverse(const float* qp, const float* kp, int64_t S, int64_t qb, int64_t kb, int64_t Pq,
                                    int64_t Pk, int64_t pd, int64_t radix, int64_t beam, float div, int32_t* out,
                                    int64_t C, int layout, void* stream) {
  SPRUCE_REQUIRE(out != nullptr, "out must be a non-null device pointer");
  SPRUCE_REQUIRE(layout == SPRUCE_KP_ROWS || layout == SPRUCE_KP_INTERLEAVED, "unknown key table layout %d", layout);
  SPRUCE_REQUIRE(kb >= 1 && kb < ((int64_t)1 << 30), "key blocks must be in [1, 2^30)");
  SPRUCE_REQUIRE(radix >= 2, "radix must be >= 2, got %lld", (long long)radix);
  SPRUCE_REQUIRE(beam >= 1, "beam must be >= 1, got %lld", (long long)beam);
  SPRUCE_REQUIRE(beam <= 32 && radix <= 64 && beam * radix <= 64,
                 "beam * radix must be <= 64, got beam %lld, radix %lld", (long long)beam, (long long)radix);
  TraverseParams p{};
  // Level counts ceil(prev / radix) down to one root; node (v, i) has ID offset[v] + i.
  int64_t count = kb, span = 1, total = 0;
  int levels = 0;
  while (true) {
    SPRUCE_REQUIRE(levels < kMaxLevels, "tree too deep");
    p.count[levels] = (int)count;
    p.offset[levels] = (int)total;
    p.span[levels] = span;
    total += count;
    ++levels;
    if (count == 1) break;
    count = (count + radix - 1) / radix;
    span *= radix;
  }
  int rc = check_score_args(qp, kp, S, qb, total, Pq, Pk, pd, div);
  if (rc) return rc;
  // Output width: the beam width after the last level.
  int64_t W = 1;
  for (int v = levels - 2; v >= 0; --v) {
    int64_t k = beam < W * radix ? beam : W * radix;
    W = k < p.count[v] ? k : p.count[v];
  }
  SPRUCE_REQUIRE(C == W, "out width must be %lld for this tree and beam, got %lld", (long long)W, (long long)C);
  const bool il = layout == SPRUCE_KP_INTERLEAVED;
  p.sc = ScoreParams2{qp, kp, S, (int)qb, (int)total, (int)Pq, (int)Pk, (int)pd, div, il ? 4 : (int)pd,
                      il ? 4 * (int)Pk : 4};
  p.kb = (int)kb;
  p.radix = (int)radix;
  p.beam = (int)beam;
  p.levels = levels;
  p.C = (int)C;
  p.out = out;
  const size_t lds = ((size_t)Pq * pd + 64 * Pk) * sizeof(float) + 3 * 64 * sizeof(int);
  const dim3 grid((unsigned)(S * qb));
  switch (Pq) {
    case 1: hipLaunchKernelGGL(tree_traverse_kernel<1>, grid, dim3(64), lds, (hipStream_t)stream, p); break;
    case 2: hipLaunchKernelGGL(tree_traverse_kernel<2>, grid, dim3(64), lds, (hipStream_t)stream, p); break;
    case 4: hipLaunchKernelGGL(tree_traverse_kernel<4>, grid, dim3(64), lds, (hipStream_t)stream, p); break;
    case 8:
      // The deployed shape (8 prototypes, p = 128) with compile-time strides.
      if (pd == 128 && il && Pk == 8)
        hipLaunchKernelGGL((tree_traverse_kernel<8, 128, 32>), grid, dim3(64), lds, (hipStream_t)stream, p);
      else if (pd == 128 && !il)
        hipLaunchKernelGGL((tree_traverse_kernel<8, 128, 4>), grid, dim3(64), lds, (hipStream_t)stream, p);
      else
        hipLaunchKernelGGL(tree_traverse_kernel<8>, grid, dim3(64), lds, (hipStream_t)stream, p);
      break;
    default: hipLaunchKernelGGL(tree_traverse_kernel<0>, grid, dim3(64), lds, (hipStream_t)stream, p); break;
  }
  return check_launch("tree_traverse_kernel");
}

extern "C" int spruce_gate_candidate_scores(const float* qp, const float* kp, const int32_t* ids, int64_t S,
                                            int64_t qb, int64_t N, int64_t C, int64_t Pq, int64_t Pk, int64_t pd,
                                            float div, float* out, void* stream) {
  int rc = check_score_args(qp, kp, S, qb, N, Pq, Pk, pd, div);
  if (rc) return rc;
  SPRUCE_REQUIRE(C >= 1 && ids != nullptr && out != nullptr, "ids and out must be non-null with C >= 1");
  CandParams p{};
  p.sc = ScoreParams2{qp, kp, S, (int)qb, (int)N, (int)Pq, (int)Pk, (int)pd, div, (int)pd, 4};
  p.ids = ids;
  p.C = (int)C;
  p.out = out;
  const size_t lds = ((size_t)Pq * pd + 64 * Pk) * sizeof(float);
  hipLaunchKernelGGL(candidate_scores_kernel, dim3((unsigned)(S * qb)), dim3(64), lds, (hipStream_t)stream, p);
  return check_launch("candidate_scores_kernel");
}
