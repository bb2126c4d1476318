// Residual-tree K/V summaries: the positional prototype means of
// build_kv_summary_table (sparse/summaries.py:52-142).
//
// For every batch b and token range r = [start, end) (one per tree node and
// prototype, computed by the host from the tree layout), with valid[b, t] the
// optional key-padding mask:
//   count[b, r]      = #valid tokens in the range
//   keys[b, h, r]    = sum_t valid * K[b, h, t] / max(count, 1)   (float32)
//   values[b, h, r]  = the same over V
//   log_counts[b, r] = log(count), or -inf when the range holds no valid token
// The reference forms the sums as differences of float32 prefix sums; here
// they are direct float32 sums (smaller rounding error, same value up to it).
//
// Two kernels.  chunk_sum: one pass over K and V writing per-64-token chunk
// sums (and valid counts) to the workspace.  range_sum: one workgroup per
// (b, h, range) adds the chunk sums of the fully covered chunks and the
// tokens of the partial chunks at either end, so upper tree levels never
// re-read K/V.  HBM-bound: K and V are read once, plus one chunk-sum read per
// covered chunk per level.
#include <math.h>

#include "common.h"

namespace spruce {
namespace {

constexpr int kChunk = 64;
constexpr int kSumThreads = 256;

struct SumParams {
  const void* k;
  const void* v;
  int64_t ks[4], vs[4];
  int B, H, T, D, dtype, nchunks, R;
  const uint8_t* valid;    // [B, T] or null (all valid)
  const int64_t* starts;   // [R]
  const int64_t* ends;     // [R]
  float* chunk;            // workspace [B, H, nchunks, 2, D]
  int* chunk_cnt;          // workspace [B, nchunks]
  float* keys;             // [B, H, R, D]
  float* values;           // [B, H, R, D]
  float* counts;           // [B, R]
  float* log_counts;       // [B, R]
};

__device__ __forceinline__ float load_elem(const void* base, int64_t e, int dtype) {
  if (dtype == SPRUCE_DTYPE_F32) return static_cast<const float*>(base)[e];
  const uint32_t bits = static_cast<const uint16_t*>(base)[e];
  return dtype == SPRUCE_DTYPE_F16 ? unpack1<true>(bits) : unpack1<false>(bits);
}

// Sum over tokens [t0, t1) of column d of tensor `which` (0 = K, 1 = V).
__device__ __forceinline__ float token_sum(const SumParams& p, int which, int b, int h, int d, int64_t t0,
                                           int64_t t1) {
  const void* x = which ? p.v : p.k;
  const int64_t* s = which ? p.vs : p.ks;
  const int64_t base = (int64_t)b * s[0] + (int64_t)h * s[1] + (int64_t)d * s[3];
  const uint8_t* valid = p.valid ? p.valid + (int64_t)b * p.T : nullptr;
  float acc = 0.0f;
  for (int64_t t = t0; t < t1; ++t) {
    if (valid && !valid[t]) continue;
    acc += load_elem(x, base + t * s[2], p.dtype);
  }
  return acc;
}

__global__ __launch_bounds__(kSumThreads) void chunk_sum_kernel(SumParams p) {
  const int c = blockIdx.x % p.nchunks;
  const int bh = blockIdx.x / p.nchunks;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t t0 = (int64_t)c * kChunk;
  const int64_t t1 = t0 + kChunk < p.T ? t0 + kChunk : p.T;
  float* out = p.chunk + (((int64_t)b * p.H + h) * p.nchunks + c) * 2 * p.D;
  for (int col = threadIdx.x; col < 2 * p.D; col += kSumThreads) {
    const int which = col / p.D, d = col - which * p.D;
    out[col] = token_sum(p, which, b, h, d, t0, t1);
  }
  if (h == 0 && threadIdx.x == 0) {
    int n = (int)(t1 - t0);
    if (p.valid) {
      n = 0;
      for (int64_t t = t0; t < t1; ++t) n += p.valid[(int64_t)b * p.T + t] != 0;
    }
    p.chunk_cnt[(int64_t)b * p.nchunks + c] = n;
  }
}

__global__ __launch_bounds__(kSumThreads) void range_sum_kernel(SumParams p) {
  __shared__ int partial[kSumThreads];
  const int r = blockIdx.x % p.R;
  const int bh = blockIdx.x / p.R;
  const int h = bh % p.H, b = bh / p.H;
  // Ranges come from caller memory: clamp them to [0, T] so a bad table can
  // only produce wrong sums, never an out-of-bounds read.
  int64_t s = p.starts[r], e = p.ends[r];
  s = s < 0 ? 0 : (s > p.T ? p.T : s);
  e = e < s ? s : (e > p.T ? p.T : e);
  // Full chunks [c0, c1); partial tokens [s, c0*64) and [c1*64, e).
  int64_t c0 = (s + kChunk - 1) / kChunk, c1 = e / kChunk;
  int64_t head_end = c0 * kChunk, tail_start = c1 * kChunk;
  if (c1 <= c0) {                       // range inside one chunk (or empty)
    c0 = c1 = 0;
    head_end = e;
    tail_start = e;
  }

  // Valid-token count: strided partial counts, then a tree reduction.
  int n = 0;
  if (p.valid) {
    const uint8_t* valid = p.valid + (int64_t)b * p.T;
    for (int64_t t = s + threadIdx.x; t < head_end; t += kSumThreads) n += valid[t] != 0;
    for (int64_t t = tail_start + threadIdx.x; t < e; t += kSumThreads) n += valid[t] != 0;
    for (int64_t c = c0 + threadIdx.x; c < c1; c += kSumThreads) n += p.chunk_cnt[(int64_t)b * p.nchunks + c];
  } else if (threadIdx.x == 0) {
    n = (int)(e - s);
  }
  partial[threadIdx.x] = n;
  __syncthreads();
  for (int w = kSumThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) partial[threadIdx.x] += partial[threadIdx.x + w];
    __syncthreads();
  }
  const int count = partial[0];
  const float denom = count > 1 ? (float)count : 1.0f;

  const float* chunks = p.chunk + ((int64_t)b * p.H + h) * p.nchunks * 2 * p.D;
  const int64_t orow = (((int64_t)b * p.H + h) * p.R + r) * p.D;
  for (int col = threadIdx.x; col < 2 * p.D; col += kSumThreads) {
    const int which = col / p.D, d = col - which * p.D;
    float acc = token_sum(p, which, b, h, d, s, head_end);
    for (int64_t c = c0; c < c1; ++c) acc += chunks[c * 2 * p.D + col];
    acc += token_sum(p, which, b, h, d, tail_start, e);
    (which ? p.values : p.keys)[orow + d] = acc / denom;
  }
  if (h == 0 && threadIdx.x == 0) {
    p.counts[(int64_t)b * p.R + r] = (float)count;
    p.log_counts[(int64_t)b * p.R + r] = count > 0 ? logf((float)count) : -__builtin_inff();
  }
}

size_t workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  const int64_t nchunks = (T + kChunk - 1) / kChunk;
  const size_t sums = (size_t)(B * H * nchunks * 2 * D) * sizeof(float);
  const size_t cnts = (size_t)(B * nchunks) * sizeof(int);
  return ((sums + 255) / 256) * 256 + cnts;
}

}  // namespace
}  // namespace spruce

using namespace spruce;

extern "C" size_t spruce_kv_summary_workspace_bytes(int64_t B, int64_t Hkv, int64_t T, int64_t D) {
  if (B < 1 || Hkv < 1 || T < 1 || D < 1) return 0;
  return workspace_bytes(B, Hkv, T, D);
}

extern "C" int spruce_kv_summary(const void* k, const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B,
                                 int64_t Hkv, int64_t T, int64_t D, int dtype, const uint8_t* valid,
                                 const int64_t* range_starts, const int64_t* range_ends, int64_t R, float* keys,
                                 float* values, float* counts, float* log_counts, void* workspace,
                                 size_t workspace_bytes_given, void* stream) {
  SPRUCE_REQUIRE(k && v && ks && vs && keys && values && counts && log_counts && workspace,
                 "tensors, strides and workspace must be non-null");
  SPRUCE_REQUIRE(range_starts && range_ends, "range tables must be non-null");
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  SPRUCE_REQUIRE(B >= 1 && Hkv >= 1 && T >= 1 && D >= 1 && R >= 1, "invalid shape");
  SPRUCE_REQUIRE(B < (1 << 20) && Hkv < (1 << 16) && T < ((int64_t)1 << 30) && D <= 4096 && R < ((int64_t)1 << 30),
                 "shape out of range");
  for (int i = 0; i < 4; ++i) SPRUCE_REQUIRE(ks[i] >= 0 && vs[i] >= 0, "negative strides are not supported");
  const size_t need = workspace_bytes(B, Hkv, T, D);
  SPRUCE_REQUIRE(workspace_bytes_given >= need, "workspace needs %zu bytes, got %zu", need, workspace_bytes_given);
  SPRUCE_REQUIRE(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  SumParams p;
  p.k = k; p.v = v;
  for (int i = 0; i < 4; ++i) { p.ks[i] = ks[i]; p.vs[i] = vs[i]; }
  p.B = (int)B; p.H = (int)Hkv; p.T = (int)T; p.D = (int)D; p.dtype = dtype;
  p.nchunks = (int)((T + kChunk - 1) / kChunk);
  p.R = (int)R;
  p.valid = valid;
  p.starts = range_starts; p.ends = range_ends;
  const size_t sums = (size_t)(B * Hkv * p.nchunks * 2 * D) * sizeof(float);
  p.chunk = static_cast<float*>(workspace);
  p.chunk_cnt = reinterpret_cast<int*>(static_cast<char*>(workspace) + ((sums + 255) / 256) * 256);
  p.keys = keys; p.values = values; p.counts = counts; p.log_counts = log_counts;
  const int64_t g1 = B * Hkv * (int64_t)p.nchunks, g2 = B * Hkv * R;
  SPRUCE_REQUIRE(g1 < ((int64_t)1 << 31) && g2 < ((int64_t)1 << 31), "too many workgroups");
  hipLaunchKernelGGL(chunk_sum_kernel, dim3((unsigned)g1), dim3(kSumThreads), 0, (hipStream_t)stream, p);
  int rc = check_launch("chunk_sum_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(range_sum_kernel, dim3((unsigned)g2), dim3(kSumThreads), 0, (hipStream_t)stream, p);
  return check_launch("range_sum_kernel");
}
