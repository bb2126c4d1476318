// Residual-tree frontiers of selected_blocks rows on gfx950.
//
// Replaces the host loops of build_residual_summary_nodes /
// residual_frontier_for_row (interfaces/residual_summaries.py:119-222): for
// every (batch, layer, KV group, query block q) row, the maximal nodes of the
// leaf-first binary key tree that cover the causal blocks [0, q] the row does
// not list, in ascending node-ID order.
//
// Characterisation used here (equivalent to the reference's top-down visit):
// call a node "blocked" when its leaf range holds a listed block or reaches
// past q.  Blocked propagates upward (a parent's range contains its
// children's), so the visit takes exactly the unblocked nodes whose parent is
// blocked (or that are the root).  One wavefront per row builds the tree's
// occupancy bits in LDS -- level 0 from the row's ids, each higher level by
// OR-ing child pairs 64 bits at a time -- then walks the levels in ID order,
// 64 nodes per step, and compacts the frontier nodes with a ballot.  Only
// nodes that start at or before q are ever touched: about 2(q+1) bits.
#include "common.h"

namespace spruce {

constexpr int kMaxTreeLevels = 32;

struct FrontierParams {
  const int32_t* sel;
  int64_t ss[5];  // [B, L, G, Qb, K] element strides
  int64_t rows;   // B * L * G * Qb
  int L, G, Qb, K;
  int levels;
  int words;                       // LDS words per row (all levels)
  int wofs[kMaxTreeLevels];        // first LDS word of each level
  int offs[kMaxTreeLevels];        // first node ID of each level
  int32_t* counts;                 // [rows]: frontier size, -1 when a listed id is > q
  int32_t* out;                    // [rows, S] or null (count only)
  int S;
};

// Even bits of x (bit 2j -> bit j): the Morton de-interleave of one lane.
__device__ __forceinline__ uint32_t even_bits(uint64_t x) {
  x &= 0x5555555555555555ull;
  x = (x | (x >> 1)) & 0x3333333333333333ull;
  x = (x | (x >> 2)) & 0x0F0F0F0F0F0F0F0Full;
  x = (x | (x >> 4)) & 0x00FF00FF00FF00FFull;
  x = (x | (x >> 8)) & 0x0000FFFF0000FFFFull;
  x = (x | (x >> 16)) & 0x00000000FFFFFFFFull;
  return (uint32_t)x;
}

__global__ __launch_bounds__(64) void residual_frontier_kernel(const FrontierParams p) {
  extern __shared__ uint32_t bits[];
  const int64_t row = blockIdx.x;
  if (row >= p.rows) return;  // uniform
  const int lane = threadIdx.x;
  const int q = (int)(row % p.Qb);
  const int64_t rest = row / p.Qb;
  const int g = (int)(rest % p.G);
  const int64_t bl = rest / p.G;
  const int l = (int)(bl % p.L);
  const int64_t b = bl / p.L;
  const int nb = q + 1;  // causal leaves [0, q]

  // Nodes of level v that start before nb: ceil(nb / 2^v).
  auto live = [&](int v) { return ((nb - 1) >> v) + 1; };

  for (int v = 0; v < p.levels; ++v) {
    // One spare word per level so the pair read of the level above stays in range.
    const int w = ((live(v) + 31) >> 5) + 1;
    for (int i = lane; i < w; i += 64) bits[p.wofs[v] + i] = 0u;
  }
  __syncthreads();

  const int32_t* srow = p.sel + b * p.ss[0] + (int64_t)l * p.ss[1] + (int64_t)g * p.ss[2] + (int64_t)q * p.ss[3];
  bool bad = false;
  for (int i = lane; i < p.K; i += 64) {
    const int id = srow[(int64_t)i * p.ss[4]];
    if (id > q) bad = true;               // non-causal id: the reference raises
    else if (id >= 0) atomicOr(&bits[id >> 5], 1u << (id & 31));
  }
  const bool any_bad = __ballot(bad) != 0;
  __syncthreads();

  for (int v = 1; v < p.levels; ++v) {
    const int w = (live(v) + 31) >> 5;
    const uint32_t* lo = bits + p.wofs[v - 1];
    for (int i = lane; i < w; i += 64) {
      const uint64_t x = (uint64_t)lo[2 * i] | ((uint64_t)lo[2 * i + 1] << 32);
      bits[p.wofs[v] + i] = even_bits(x | (x >> 1));
    }
    __syncthreads();
  }

  int count = 0;
  int32_t* orow = p.out ? p.out + row * (int64_t)p.S : nullptr;
  if (!any_bad) {
    for (int v = 0; v < p.levels; ++v) {
      const int n = live(v);
      const uint32_t* lv = bits + p.wofs[v];
      const uint32_t* up = v + 1 < p.levels ? bits + p.wofs[v + 1] : nullptr;
      for (int base = 0; base < n; base += 64) {
        const int i = base + lane;
        bool emit = false;
        if (i < n) {
          int end = (i + 1) << v;
          end = end < p.Qb ? end : p.Qb;
          const bool blocked = ((lv[i >> 5] >> (i & 31)) & 1u) || end > nb;
          bool pblocked = true;  // the root has no parent
          if (up) {
            const int pi = i >> 1;
            int pend = (pi + 1) << (v + 1);
            pend = pend < p.Qb ? pend : p.Qb;
            pblocked = ((up[pi >> 5] >> (pi & 31)) & 1u) || pend > nb;
          }
          emit = !blocked && pblocked;
        }
        const uint64_t m = __ballot(emit);
        if (emit && orow) {
          const int pos = count + __builtin_popcountll(m & ((1ull << lane) - 1ull));
          if (pos < p.S) orow[pos] = p.offs[v] + i;
        }
        count += __builtin_popcountll(m);
      }
    }
  }
  if (orow)
    for (int j = count + lane; j < p.S; j += 64) orow[j] = -1;
  if (lane == 0) p.counts[row] = any_bad ? -1 : count;
}

}  // namespace spruce

using namespace spruce;

extern "C" int spruce_residual_frontier(const int32_t* selected, const int64_t ss[5], int64_t B, int64_t L,
                                        int64_t G, int64_t Qb, int64_t K, int32_t* counts, int32_t* out,
                                        int64_t S, void* stream) {
  SPRUCE_REQUIRE(selected != nullptr || K == 0, "selected must be a non-null device pointer");
  SPRUCE_REQUIRE(ss != nullptr, "stride array must be non-null");
  SPRUCE_REQUIRE(counts != nullptr, "counts must be a non-null device pointer");
  SPRUCE_REQUIRE(B >= 0 && L >= 0 && G >= 0 && K >= 0 && S >= 0, "sizes must be non-negative");
  SPRUCE_REQUIRE(Qb >= 1 && Qb <= (1 << 20), "query blocks must be in [1, 2^20], got %lld", (long long)Qb);
  SPRUCE_REQUIRE(out != nullptr || S == 0, "out must be non-null when S > 0");
  FrontierParams p{};
  p.sel = selected;
  for (int i = 0; i < 5; ++i) p.ss[i] = ss[i];
  p.rows = B * L * G * Qb;
  SPRUCE_REQUIRE(p.rows < ((int64_t)1 << 31), "too many rows");
  p.L = (int)(L > 0 ? L : 1);
  p.G = (int)(G > 0 ? G : 1);
  p.Qb = (int)Qb;
  p.K = (int)K;
  // Level counts ceil(prev / 2) down to one root (interfaces/residual_summaries.py:72-80).
  int count = (int)Qb, levels = 0, words = 0, node = 0;
  while (true) {
    p.wofs[levels] = words;
    p.offs[levels] = node;
    words += (count + 31) / 32 + 1;
    node += count;
    ++levels;
    if (count == 1) break;
    count = (count + 1) / 2;
  }
  p.levels = levels;
  p.words = words;
  p.counts = counts;
  p.out = out;
  p.S = (int)S;
  const size_t lds = (size_t)words * 4;
  SPRUCE_REQUIRE(lds <= 64 * 1024, "tree too large for one workgroup's LDS (%zu bytes)", lds);
  if (p.rows == 0) return SPRUCE_OK;
  hipLaunchKernelGGL(residual_frontier_kernel, dim3((unsigned)p.rows), dim3(64), lds, (hipStream_t)stream, p);
  return check_launch("residual_frontier_kernel");
}
