// Route packing into the selected_blocks contract (int32 rows, ascending,
// PAD = -1).  Two policies, both from scripts/export_selected_blocks.py:
//
//   pack_ids   selected_ids_to_blocks (:79-175): forced sink blocks, then the
//              smallest distinct causal non-local traversal IDs that fit the
//              budget, then the local window {q-lw .. q}.
//   pack_mask  selected_mask_to_blocks (:37-76): the first non-local causal
//              columns of a boolean row that fit, then the local window.
//
// The three groups are disjoint and ordered (sink < sink_blocks <= non-local <
// q - lw <= local), so the sorted row the reference builds with a sentinel
// sort is their concatenation.  One wavefront per row; HBM-bound integer work.
#include "common.h"

namespace spruce {
namespace {

constexpr int kPackWaves = 4;
constexpr int kPackMaxKb = 65536;                 // bitmap: 2048 words per wave
constexpr int kPackWords = kPackMaxKb / 32;

__device__ __forceinline__ uint64_t lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Inclusive wave prefix sum of v (64 lanes) through LDS-free DPP-less shuffles.
__device__ __forceinline__ int wave_inclusive_sum(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Writes the local window q-lw..q (ids >= 0; with check_kb also < kb) at
// out[pos...], then pads the row with -1 up to width W.
__device__ __forceinline__ void finish_row(int32_t* row, int pos, int q, int lw, int kb, bool check_kb, int W,
                                           int lane) {
  const int lo = q - lw < 0 ? 0 : q - lw;
  const int hi = check_kb ? (q < kb - 1 ? q : kb - 1) : q;
  const int nloc = hi >= lo ? hi - lo + 1 : 0;
  for (int j = lane; j < W - pos; j += 64) row[pos + j] = j < nloc ? lo + j : -1;
}

template <typename Id>
__global__ __launch_bounds__(64 * kPackWaves) void pack_ids_kernel(const Id* __restrict__ ids, int64_t R, int qb,
                                                                     int C, int kb, int K, int lw, int sink,
                                                                     int32_t* __restrict__ out, int W) {
  __shared__ uint32_t bitmap[kPackWaves][kPackWords];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * kPackWaves + wave;
  if (r >= R) return;                               // whole wave leaves together; no block barrier follows
  const int q = (int)(r % qb);
  uint32_t* bm = bitmap[wave];
  int32_t* row = out + r * W;

  const int local_count = (q + 1) < (lw + 1) ? (q + 1) : (lw + 1);
  int sink_count = q - lw;
  sink_count = sink_count < 0 ? 0 : (sink_count > sink ? sink : sink_count);
  const int remaining = K - local_count - sink_count;

  // Candidate IDs: sink <= id < min(q - lw, kb) (id <= q follows).
  const int lo = sink;
  int hi = q - lw < kb ? q - lw : kb;
  const int span = hi > lo ? hi - lo : 0;
  const int nwords = (span + 31) >> 5;

  for (int w = lane; w < nwords; w += 64) bm[w] = 0u;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  const Id* src = ids + r * C;
  for (int c = lane; c < C; c += 64) {
    const int64_t id = (int64_t)src[c];
    if (id >= lo && id < hi) {
      const int off = (int)(id - lo);
      atomicOr(&bm[off >> 5], 1u << (off & 31));
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  __builtin_amdgcn_wave_barrier();

  for (int j = lane; j < sink_count; j += 64) row[j] = j;
  int emitted = 0;
  const int budget = remaining;
  for (int base = 0; base < nwords && emitted < budget; base += 64) {
    const int w = base + lane;
    uint32_t bits = w < nwords ? bm[w] : 0u;
    const int cnt = __popc(bits);
    const int incl = wave_inclusive_sum(cnt, lane);
    int p = emitted + incl - cnt;
    while (bits && p < budget) {
      const int b = __ffs(bits) - 1;
      bits &= bits - 1;
      row[sink_count + p] = lo + (w << 5) + b;
      ++p;
    }
    emitted += __shfl(incl, 63, 64);
  }
  if (emitted > budget) emitted = budget;
  finish_row(row, sink_count + emitted, q, lw, kb, false, W, lane);
}

__global__ __launch_bounds__(64 * kPackWaves) void pack_mask_kernel(const uint8_t* __restrict__ mask, int64_t R,
                                                                      int qb, int kb, int K, int lw,
                                                                      int32_t* __restrict__ out, int W) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kPackWaves + (threadIdx.x >> 6);
  if (r >= R) return;
  const int q = (int)(r % qb);
  int32_t* row = out + r * W;
  const int lo = q - lw < 0 ? 0 : q - lw;
  const int hi = q < kb - 1 ? q : kb - 1;
  const int local_count = hi >= lo ? hi - lo + 1 : 0;
  const int budget = K - local_count;
  // Non-local causal columns: j < min(q - lw, kb).
  const int end = q - lw < kb ? q - lw : kb;
  const uint8_t* src = mask + r * (int64_t)kb;
  int emitted = 0;
  for (int base = 0; base < end && emitted < budget; base += 64) {
    const int j = base + lane;
    const bool on = j < end && src[j] != 0;
    const uint64_t ball = __ballot(on);
    const int p = emitted + __popcll(ball & lanes_below(lane));
    if (on && p < budget) row[p] = j;
    emitted += __popcll(ball);
  }
  if (emitted > budget) emitted = budget;
  finish_row(row, emitted, q, lw, kb, true, W, lane);
}

}  // namespace
}  // namespace spruce

using namespace spruce;

extern "C" int spruce_pack_selected_ids(const void* ids, int id_bytes, int64_t R, int64_t qb, int64_t C,
                                        int64_t key_blocks, int64_t k_selected, int64_t local_window,
                                        int64_t sink_blocks, int32_t* out, int64_t out_cols, void* stream) {
  SPRUCE_REQUIRE(out, "out must be non-null");
  SPRUCE_REQUIRE(id_bytes == 4 || id_bytes == 8, "id_bytes must be 4 or 8, got %d", id_bytes);
  SPRUCE_REQUIRE(R >= 0 && qb >= 1 && C >= 0, "invalid ids shape");
  SPRUCE_REQUIRE(R % qb == 0, "rows (%lld) must be a multiple of query blocks (%lld)", (long long)R,
                 (long long)qb);
  SPRUCE_REQUIRE(k_selected >= 1, "k_selected must be >= 1, got %lld", (long long)k_selected);
  SPRUCE_REQUIRE(local_window >= 0, "local_window must be >= 0, got %lld", (long long)local_window);
  SPRUCE_REQUIRE(sink_blocks >= 0, "sink_blocks must be >= 0, got %lld", (long long)sink_blocks);
  SPRUCE_REQUIRE(k_selected >= local_window + 1 + sink_blocks,
                 "k_selected=%lld cannot fit local window size %lld plus %lld sink block(s)",
                 (long long)k_selected, (long long)(local_window + 1), (long long)sink_blocks);
  SPRUCE_REQUIRE(key_blocks >= 1, "key_blocks must be >= 1, got %lld", (long long)key_blocks);
  SPRUCE_REQUIRE(key_blocks <= kPackMaxKb, "at most %d key blocks are supported, got %lld", kPackMaxKb,
                 (long long)key_blocks);
  SPRUCE_REQUIRE(qb < ((int64_t)1 << 30) && C < ((int64_t)1 << 30) && k_selected < ((int64_t)1 << 30),
                 "sizes out of range");
  const int64_t sink = sink_blocks < key_blocks ? sink_blocks : key_blocks;
  const int64_t width = C + sink + local_window + 1;
  const int64_t W = k_selected < width ? k_selected : width;
  SPRUCE_REQUIRE(out_cols == W, "out must have %lld columns, got %lld", (long long)W, (long long)out_cols);
  if (R == 0) return SPRUCE_OK;
  SPRUCE_REQUIRE(ids || C == 0, "ids must be non-null");
  const int64_t grid = (R + kPackWaves - 1) / kPackWaves;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "too many rows");
  if (id_bytes == 4)
    hipLaunchKernelGGL(pack_ids_kernel<int32_t>, dim3((unsigned)grid), dim3(64 * kPackWaves), 0,
                       (hipStream_t)stream, (const int32_t*)ids, R, (int)qb, (int)C, (int)key_blocks,
                       (int)k_selected, (int)local_window, (int)sink, out, (int)W);
  else
    hipLaunchKernelGGL(pack_ids_kernel<int64_t>, dim3((unsigned)grid), dim3(64 * kPackWaves), 0,
                       (hipStream_t)stream, (const int64_t*)ids, R, (int)qb, (int)C, (int)key_blocks,
                       (int)k_selected, (int)local_window, (int)sink, out, (int)W);
  return check_launch("pack_ids_kernel");
}

extern "C" int spruce_pack_selected_mask(const uint8_t* mask, int64_t R, int64_t qb, int64_t kb,
                                         int64_t k_selected, int64_t local_window, int32_t* out,
                                         int64_t out_cols, void* stream) {
  SPRUCE_REQUIRE(out, "out must be non-null");
  SPRUCE_REQUIRE(R >= 0 && qb >= 1 && kb >= 1, "invalid mask shape");
  SPRUCE_REQUIRE(R % qb == 0, "rows (%lld) must be a multiple of query blocks (%lld)", (long long)R,
                 (long long)qb);
  SPRUCE_REQUIRE(k_selected >= 1, "k_selected must be >= 1, got %lld", (long long)k_selected);
  SPRUCE_REQUIRE(local_window >= 0, "local_window must be >= 0, got %lld", (long long)local_window);
  SPRUCE_REQUIRE(k_selected >= local_window + 1, "k_selected=%lld cannot fit local window size %lld",
                 (long long)k_selected, (long long)(local_window + 1));
  SPRUCE_REQUIRE(qb < ((int64_t)1 << 30) && kb < ((int64_t)1 << 30) && k_selected < ((int64_t)1 << 30),
                 "sizes out of range");
  const int64_t W = k_selected < kb ? k_selected : kb;
  SPRUCE_REQUIRE(out_cols == W, "out must have %lld columns, got %lld", (long long)W, (long long)out_cols);
  if (R == 0) return SPRUCE_OK;
  SPRUCE_REQUIRE(mask, "mask must be non-null");
  const int64_t grid = (R + kPackWaves - 1) / kPackWaves;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "too many rows");
  hipLaunchKernelGGL(pack_mask_kernel, dim3((unsigned)grid), dim3(64 * kPackWaves), 0, (hipStream_t)stream, mask,
                     R, (int)qb, (int)kb, (int)k_selected, (int)local_window, out, (int)W);
  return check_launch("pack_mask_kernel");
}
