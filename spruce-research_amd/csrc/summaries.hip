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
// chunk_sum: one pass over K and V writing per-64-token chunk sums (and valid
// counts) to the workspace.  For 16-byte-aligned rows (the usual case) a
// float64 exclusive prefix of the chunk sums follows, and range_sum adds, per
// (b, h, range), the prefix difference over the fully covered chunks and the
// tokens of the partial chunks at either end (16-byte loads, LDS reduction):
// upper tree levels never re-read K/V and each range costs O(1) chunk reads.
// Other layouts take a scalar path that adds the covered chunk sums one by
// one.  HBM-bound: K and V are read about twice (once for the chunk sums,
// once more for the within-chunk ranges of the two lowest tree levels).
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
  // Eight independent partial sums keep eight loads in flight; they are
  // combined pairwise at the end.
  float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t t = t0;
  for (; t + 8 <= t1; t += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float v = load_elem(x, base + (t + u) * s[2], p.dtype);
      part[u] += (valid && !valid[t + u]) ? 0.0f : v;
    }
  }
  for (int u = 0; t < t1; ++t, ++u) {
    const float v = load_elem(x, base + t * s[2], p.dtype);
    part[u] += (valid && !valid[t]) ? 0.0f : v;
  }
  return ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
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
    float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t c = c0;
    for (; c + 8 <= c1; c += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) part[u] += chunks[(c + u) * 2 * p.D + col];
    }
    for (int u = 0; c < c1; ++c, ++u) part[u] += chunks[c * 2 * p.D + col];
    acc += ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
    acc += token_sum(p, which, b, h, d, tail_start, e);
    (which ? p.values : p.keys)[orow + d] = acc / denom;
  }
  if (h == 0 && threadIdx.x == 0) {
    p.counts[(int64_t)b * p.R + r] = (float)count;
    p.log_counts[(int64_t)b * p.R + r] = count > 0 ? logf((float)count) : -__builtin_inff();
  }
}

// ---------------------------------------------------------------- vector path
// For 16-byte-aligned rows with a contiguous last dim and D % 8 == 0: thread
// (r, gc) = (tid / 16, tid % 16) reads 16 bytes (8 columns) of token rows
// r, r + 16, ... and of granule-columns gc, gc + 16, ... over [K | V]; the 16
// token lanes are then reduced through LDS.  Full 64-token chunks inside a
// range come from float64 prefix sums of the chunk sums (two reads per range).
constexpr int kMaxGranCols = 64;   // 2 * D / 8 for D <= 256

struct VecParams {
  SumParams p;
  double* prefix;     // [B, H, nchunks + 1, 2D] exclusive prefix of chunk sums
  int* cnt_prefix;    // [B, nchunks + 1]
};

// Adds 8 columns of token t (tensor which, granule gi) into a[0..8).
__device__ __forceinline__ void add_row8(const SumParams& p, int which, int b, int h, int gi, int64_t t, float* a) {
  const void* x = which ? p.v : p.k;
  const int64_t* st = which ? p.vs : p.ks;
  float v[8];
  load8f(x, (int64_t)b * st[0] + (int64_t)h * st[1] + t * st[2] + 8 * gi, p.dtype, v);
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] += v[e];
}

// Sums tokens tok(i), i in [0, n), over all 2D columns into out[0 .. 2D) (LDS).
template <typename TokOf>
__device__ __forceinline__ void vec_token_sums(const SumParams& p, int b, int h, int n, TokOf tok, float* red,
                                               float* out) {
  const int r = threadIdx.x >> 4, gl = threadIdx.x & 15;
  const int G = p.D / 8, GC = 2 * G;
  float acc[kMaxGranCols / 16][8];
#pragma unroll
  for (int k = 0; k < kMaxGranCols / 16; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;
  const uint8_t* valid = p.valid ? p.valid + (int64_t)b * p.T : nullptr;
  for (int i = r; i < n; i += 16) {
    const int64_t t = tok(i);
    if (valid && !valid[t]) continue;
#pragma unroll
    for (int k = 0; k < kMaxGranCols / 16; ++k) {
      const int gc = gl + 16 * k;
      if (gc < GC) add_row8(p, gc >= G, b, h, gc >= G ? gc - G : gc, t, acc[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < kMaxGranCols / 16; ++k) {
    const int gc = gl + 16 * k;
    if (gc < GC)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[r * 2 * p.D + 8 * gc + e] = acc[k][e];
  }
  __syncthreads();
  for (int col = threadIdx.x; col < 2 * p.D; col += kSumThreads) {
    float sum = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) sum += red[rr * 2 * p.D + col];
    out[col] = sum;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kSumThreads) void chunk_sum_vec_kernel(SumParams p) {
  extern __shared__ float lds[];
  float* red = lds;                  // [16][2D]
  float* out = lds + 16 * 2 * p.D;   // [2D]
  const int c = blockIdx.x % p.nchunks;
  const int bh = blockIdx.x / p.nchunks;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t t0 = (int64_t)c * kChunk;
  const int n = (int)((t0 + kChunk < p.T ? t0 + kChunk : p.T) - t0);
  vec_token_sums(p, b, h, n, [&](int i) { return t0 + i; }, red, out);
  float* dst = p.chunk + (((int64_t)b * p.H + h) * p.nchunks + c) * 2 * p.D;
  for (int col = threadIdx.x; col < 2 * p.D; col += kSumThreads) dst[col] = out[col];
  if (h == 0 && threadIdx.x == 0) {
    int cnt = n;
    if (p.valid) {
      cnt = 0;
      for (int i = 0; i < n; ++i) cnt += p.valid[(int64_t)b * p.T + t0 + i] != 0;
    }
    p.chunk_cnt[(int64_t)b * p.nchunks + c] = cnt;
  }
}

// Exclusive float64 prefix over the chunk sums.  A workgroup covers one
// (b, h) and 16 columns; its 256 threads split the chunks into 16 segments:
// segment sums, their prefix in LDS, then each segment's running prefix.
constexpr int kScanCols = 16, kScanSegs = 16;
__global__ __launch_bounds__(kSumThreads) void chunk_prefix_kernel(VecParams vp) {
  const SumParams& p = vp.p;
  __shared__ double segsum[kScanSegs][kScanCols];
  const int ncg = (2 * p.D + kScanCols - 1) / kScanCols;
  const int bh = blockIdx.x / ncg, cg = blockIdx.x % ncg;
  const int b = bh / p.H, h = bh % p.H;
  const int cl = threadIdx.x % kScanCols, sg = threadIdx.x / kScanCols;
  const int col = cg * kScanCols + cl;
  const bool on = col < 2 * p.D;
  const int per = (p.nchunks + kScanSegs - 1) / kScanSegs;
  const int c0 = sg * per, c1 = c0 + per < p.nchunks ? c0 + per : p.nchunks;
  const float* src = p.chunk + (int64_t)bh * p.nchunks * 2 * p.D;
  double* dst = vp.prefix + (int64_t)bh * (p.nchunks + 1) * 2 * p.D;
  double sum = 0.0;
  if (on)
    for (int c = c0; c < c1; ++c) sum += (double)src[(int64_t)c * 2 * p.D + col];
  segsum[sg][cl] = sum;
  __syncthreads();
  double run = 0.0;
  for (int q = 0; q < sg; ++q) run += segsum[q][cl];
  if (on) {
    if (sg == 0) dst[col] = 0.0;
    for (int c = c0; c < c1; ++c) {
      run += (double)src[(int64_t)c * 2 * p.D + col];
      dst[(int64_t)(c + 1) * 2 * p.D + col] = run;
    }
  }
  // Valid-token count prefix (only read when a padding mask is given): one
  // workgroup per batch row, 256 segments of chunks, same three steps.
  if (p.valid && h == 0 && cg == 0) {
    __shared__ int cseg[kSumThreads];
    const int cper = (p.nchunks + kSumThreads - 1) / kSumThreads;
    const int d0 = threadIdx.x * cper, d1 = d0 + cper < p.nchunks ? d0 + cper : p.nchunks;
    const int* cc = p.chunk_cnt + (int64_t)b * p.nchunks;
    int* cp = vp.cnt_prefix + (int64_t)b * (p.nchunks + 1);
    int seg = 0;
    for (int c = d0; c < d1; ++c) seg += cc[c];
    cseg[threadIdx.x] = seg;
    __syncthreads();
    int acc = 0;
    for (int q = 0; q < (int)threadIdx.x; ++q) acc += cseg[q];
    if (threadIdx.x == 0) cp[0] = 0;
    for (int c = d0; c < d1; ++c) {
      acc += cc[c];
      cp[c + 1] = acc;
    }
  }
}

// One wavefront per (b, h, range): lane = (token lane r = lane / 16, granule
// lane gl = lane % 16); the 4 token lanes are combined with cross-lane
// shuffles, so the kernel uses no LDS and no barriers.
__global__ __launch_bounds__(kSumThreads) void range_sum_vec_kernel(VecParams vp) {
  const SumParams& p = vp.p;
  const int lane = threadIdx.x & 63;
  const int64_t idx = (int64_t)blockIdx.x * (kSumThreads / 64) + (threadIdx.x >> 6);
  if (idx >= (int64_t)p.B * p.H * p.R) return;  // whole wavefront
  const int r = (int)(idx % p.R);
  const int bh = (int)(idx / p.R);
  const int h = bh % p.H, b = bh / p.H;
  int64_t s = p.starts[r], e = p.ends[r];
  s = s < 0 ? 0 : (s > p.T ? p.T : s);
  e = e < s ? s : (e > p.T ? p.T : e);
  int64_t c0 = (s + kChunk - 1) / kChunk, c1 = e / kChunk;
  int64_t head_end = c0 * kChunk, tail_start = c1 * kChunk;
  if (c1 <= c0) {
    c0 = c1 = 0;
    head_end = e;
    tail_start = e;
  }
  const int nh = (int)(head_end - s), nt = (int)(e - tail_start);
  const int tl = lane >> 4, gl = lane & 15;
  const int G = p.D / 8, GC = 2 * G;
  constexpr int KG = kMaxGranCols / 16;
  float acc[KG][8];
#pragma unroll
  for (int k = 0; k < KG; ++k)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[k][q] = 0.f;
  const uint8_t* valid = p.valid ? p.valid + (int64_t)b * p.T : nullptr;
  int nvalid = 0;
  for (int i = tl; i < nh + nt; i += 4) {
    const int64_t t = i < nh ? s + i : tail_start + (i - nh);
    if (valid && !valid[t]) continue;
    ++nvalid;
#pragma unroll
    for (int k = 0; k < KG; ++k) {
      const int gc = gl + 16 * k;
      if (gc < GC) add_row8(p, gc >= G, b, h, gc >= G ? gc - G : gc, t, acc[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < KG; ++k)
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      acc[k][q] += __shfl_xor(acc[k][q], 16, 64);
      acc[k][q] += __shfl_xor(acc[k][q], 32, 64);
    }
  int count = (int)(e - s);
  if (valid) {
    // nvalid counts each token once per granule lane group: take lane gl = 0's.
    int n = gl == 0 ? nvalid : 0;
    n += __shfl_xor(n, 16, 64);
    n += __shfl_xor(n, 32, 64);
    n = __shfl(n, 0, 64);
    const int* cp = vp.cnt_prefix + (int64_t)b * (p.nchunks + 1);
    count = n + (c1 > c0 ? cp[c1] - cp[c0] : 0);
  }
  const float denom = count > 1 ? (float)count : 1.0f;
  const double* pre = vp.prefix + (int64_t)bh * (p.nchunks + 1) * 2 * p.D;
  const int64_t orow = (((int64_t)b * p.H + h) * p.R + r) * p.D;
  if (tl == 0) {
#pragma unroll
    for (int k = 0; k < KG; ++k) {
      const int gc = gl + 16 * k;
      if (gc >= GC) continue;
      const int which = gc >= G, d0 = 8 * (which ? gc - G : gc);
      float* o = (which ? p.values : p.keys) + orow + d0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float v = acc[k][q];
        const int col = 8 * gc + q;
        if (c1 > c0) v += (float)(pre[c1 * 2 * p.D + col] - pre[c0 * 2 * p.D + col]);
        o[q] = v / denom;
      }
    }
  }
  if (h == 0 && lane == 0) {
    p.counts[(int64_t)b * p.R + r] = (float)count;
    p.log_counts[(int64_t)b * p.R + r] = count > 0 ? logf((float)count) : -__builtin_inff();
  }
}

size_t workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  const int64_t nchunks = (T + kChunk - 1) / kChunk;
  const size_t sums = (size_t)(B * H * nchunks * 2 * D) * sizeof(float);
  const size_t cnts = (size_t)(B * nchunks) * sizeof(int);
  const size_t pre = (size_t)(B * H * (nchunks + 1) * 2 * D) * sizeof(double);
  const size_t cpre = (size_t)(B * (nchunks + 1)) * sizeof(int);
  auto up = [](size_t x) { return ((x + 255) / 256) * 256; };
  return up(sums) + up(cnts) + up(pre) + cpre;
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
  auto up = [](size_t x) { return ((x + 255) / 256) * 256; };
  const size_t sums = (size_t)(B * Hkv * p.nchunks * 2 * D) * sizeof(float);
  const size_t cnts = (size_t)(B * p.nchunks) * sizeof(int);
  const size_t pre = (size_t)(B * Hkv * (p.nchunks + 1) * 2 * D) * sizeof(double);
  char* ws = static_cast<char*>(workspace);
  p.chunk = reinterpret_cast<float*>(ws);
  p.chunk_cnt = reinterpret_cast<int*>(ws + up(sums));
  p.keys = keys; p.values = values; p.counts = counts; p.log_counts = log_counts;
  const int64_t g1 = B * Hkv * (int64_t)p.nchunks, g2 = B * Hkv * R;
  SPRUCE_REQUIRE(g1 < ((int64_t)1 << 31) && g2 < ((int64_t)1 << 31), "too many workgroups");
  const int eb = dtype == SPRUCE_DTYPE_F32 ? 4 : 2;
  const bool vec = D % 8 == 0 && 2 * D / 8 <= kMaxGranCols && ks[3] == 1 && vs[3] == 1 &&
                   ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 && (ks[0] * eb) % 16 == 0 &&
                   (ks[1] * eb) % 16 == 0 && (ks[2] * eb) % 16 == 0 && (vs[0] * eb) % 16 == 0 &&
                   (vs[1] * eb) % 16 == 0 && (vs[2] * eb) % 16 == 0;
  if (!vec) {
    hipLaunchKernelGGL(chunk_sum_kernel, dim3((unsigned)g1), dim3(kSumThreads), 0, (hipStream_t)stream, p);
    int rc = check_launch("chunk_sum_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(range_sum_kernel, dim3((unsigned)g2), dim3(kSumThreads), 0, (hipStream_t)stream, p);
    return check_launch("range_sum_kernel");
  }
  VecParams vp;
  vp.p = p;
  vp.prefix = reinterpret_cast<double*>(ws + up(sums) + up(cnts));
  vp.cnt_prefix = reinterpret_cast<int*>(ws + up(sums) + up(cnts) + up(pre));
  const size_t lds = (size_t)(17 * 2 * D) * sizeof(float);
  hipLaunchKernelGGL(chunk_sum_vec_kernel, dim3((unsigned)g1), dim3(kSumThreads), lds, (hipStream_t)stream, vp.p);
  int rc = check_launch("chunk_sum_vec_kernel");
  if (rc) return rc;
  const int64_t ncg = (2 * D + kScanCols - 1) / kScanCols;
  hipLaunchKernelGGL(chunk_prefix_kernel, dim3((unsigned)(B * Hkv * ncg)), dim3(kSumThreads), 0, (hipStream_t)stream,
                     vp);
  rc = check_launch("chunk_prefix_kernel");
  if (rc) return rc;
  const int64_t g3 = (g2 + kSumThreads / 64 - 1) / (kSumThreads / 64);
  hipLaunchKernelGGL(range_sum_vec_kernel, dim3((unsigned)g3), dim3(kSumThreads), 0, (hipStream_t)stream, vp);
  return check_launch("range_sum_vec_kernel");
}
