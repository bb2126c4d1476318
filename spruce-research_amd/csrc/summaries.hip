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
// they are float32 sums over a dyadic table (pairwise, so the rounding error
// grows with log2 of the range length rather than with the position in the
// sequence).
//
// Aligned rows (16-byte rows, contiguous last dim, D % 64 == 0, the usual case):
// pyramid_kernel reads K and V once and builds the dyadic table (16-token
// leaves, each level the pairwise sums of the one below) in the workspace,
// pyramid_top_kernel forms the small upper levels in one launch, and
// range_pyr_kernel adds, per (b, h, range), the partial leaves at the range
// ends and the table entries covering the rest: one entry for a tree-node
// prototype range.  Other layouts take a scalar path: per-64-token chunk sums, then each
// range adds its covered chunks one by one.  HBM-bound: K and V are read once.
#include <math.h>

#include <mutex>

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

// ---------------------------------------------------------------- dyadic path
// For 16-byte-aligned rows with a contiguous last dim and D % 64 == 0 the sums
// come from a dyadic table over the sequence: level 0 entry i holds the float32
// sums of tokens [16i, 16i + 16) over all 2D columns of [K | V], and level j
// entry i = level j-1 entries 2i + 2i+1, i.e. tokens [16 * 2^j * i,
// 16 * 2^j * (i + 1)).  A range is split into the partial 16-token leaves at
// its ends and the canonical dyadic cover of the whole leaves between them;
// a tree-node prototype range (aligned to its own power-of-two size) is a
// single table entry.  K/V are read once; every range costs one table row.
constexpr int kLeaf = 16;          // tokens per level-0 entry
constexpr int kFold = 4;           // levels added per launch: 16 rows -> 1
constexpr int kMaxLevels = 32;

struct PyrParams {
  SumParams p;
  float* pyr;                // [B, H, E, 2D]
  int* pcnt;                 // [B, E] valid counts (only with a mask)
  int E;                     // table entries per (b, h)
  int levels;
  int off[kMaxLevels];       // first entry of each level
  int n[kMaxLevels];         // entries of each level
};

// Entries per level for T tokens; returns the level count.
int table_levels(int64_t T, int64_t* n, int64_t* off, int64_t* E) {
  int L = 0;
  int64_t m = (T + kLeaf - 1) / kLeaf, o = 0;
  for (;;) {
    if (n) n[L] = m;
    if (off) off[L] = o;
    o += m;
    ++L;
    if (m == 1) break;
    m = (m + 1) / 2;
  }
  if (E) *E = o;
  return L;
}

// 8 columns (one 16-byte granule of 16-bit data, two of float32) of a row.
template <typename In>
struct Raw8 {
  uint4 w[In::bytes / 2];
};

template <typename In>
__device__ __forceinline__ Raw8<In> ld8(const char* p) {
  Raw8<In> r;
#pragma unroll
  for (int i = 0; i < In::bytes / 2; ++i) r.w[i] = reinterpret_cast<const uint4*>(p)[i];
  return r;
}

template <typename In>
__device__ __forceinline__ void add8(const Raw8<In>& r, float* a) {
  if constexpr (In::code == SPRUCE_DTYPE_F32) {
    a[0] += __uint_as_float(r.w[0].x); a[1] += __uint_as_float(r.w[0].y);
    a[2] += __uint_as_float(r.w[0].z); a[3] += __uint_as_float(r.w[0].w);
    a[4] += __uint_as_float(r.w[1].x); a[5] += __uint_as_float(r.w[1].y);
    a[6] += __uint_as_float(r.w[1].z); a[7] += __uint_as_float(r.w[1].w);
  } else {
    constexpr bool F16 = In::code == SPRUCE_DTYPE_F16;
    const uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] += unpack1<F16>(w[i] & 0xffffu);
      a[2 * i + 1] += unpack1<F16>(w[i] >> 16);
    }
  }
}

__device__ __forceinline__ void add_f8(const float* src, float* a) {
  const float4 x = reinterpret_cast<const float4*>(src)[0];
  const float4 y = reinterpret_cast<const float4*>(src)[1];
  a[0] += x.x; a[1] += x.y; a[2] += x.z; a[3] += x.w;
  a[4] += y.x; a[5] += y.y; a[6] += y.z; a[7] += y.w;
}

// Granule columns of [K | V]: gc in [0, 2D/8), K for gc < D/8.  Lane gl owns
// gc = gl + 16k, k < NK, with 16 * NK == 2D/8 (D % 64 == 0), so every lane is
// active for every k.  row[k] points at token 0 of its column, step[k] is the
// token stride in bytes.
template <typename In, int NK>
__device__ __forceinline__ void granule_ptrs(const SumParams& p, int b, int h, int gl, const char** row,
                                             int64_t* step) {
  const int G = p.D / 8;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int gc = gl + 16 * k;
    const bool isv = gc >= G;
    const int64_t* st = isv ? p.vs : p.ks;
    const char* base = static_cast<const char*>(isv ? p.v : p.k);
    row[k] = base + ((int64_t)b * st[0] + (int64_t)h * st[1] + 8 * (isv ? gc - G : gc)) * In::bytes;
    step[k] = st[2] * In::bytes;
  }
}

// One workgroup per (b, h, segment of 16 entries of level `base`).  With
// src < 0 the entries are level 0, summed from tokens (thread (r, gl) =
// (tid / 16, tid % 16) adds the 16 tokens of entry r in order, 16 bytes per
// granule column) and written; otherwise they are read from level src.  The
// next kFold levels are then formed by pairwise sums in LDS.
template <typename In, int NK>
__global__ __launch_bounds__(kSumThreads) void pyramid_kernel(PyrParams pp, int src) {
  extern __shared__ float lds[];
  const SumParams& p = pp.p;
  const int W = 2 * p.D;
  float* buf[2] = {lds, lds + 16 * W};            // [16][W] and [8][W]
  int* cbuf[2] = {reinterpret_cast<int*>(lds + 24 * W), reinterpret_cast<int*>(lds + 24 * W) + 16};
  const int base = src < 0 ? 0 : src;
  const int nbase = pp.n[base];
  const int nseg = (nbase + 15) / 16;
  const int seg = blockIdx.x % nseg;
  const int bh = blockIdx.x / nseg;
  const int h = bh % p.H, b = bh / p.H;
  const int r = threadIdx.x >> 4, gl = threadIdx.x & 15;
  const bool counts = pp.pcnt != nullptr && h == 0;
  float* table = pp.pyr + (int64_t)bh * pp.E * W;
  const int e = seg * 16 + r;
  float acc[NK][8];
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[k][q] = 0.f;
  int cnt = 0;
  if (e < nbase) {
    if (src < 0) {
      const int64_t t0 = (int64_t)e * kLeaf;
      const int64_t t1 = t0 + kLeaf < p.T ? t0 + kLeaf : p.T;
      const uint8_t* valid = p.valid ? p.valid + (int64_t)b * p.T : nullptr;
      const char* row[NK];
      int64_t step[NK];
      granule_ptrs<In, NK>(p, b, h, gl, row, step);
      if (!valid && t1 - t0 == kLeaf) {
        // All loads of a batch are issued before the first add (about 64
        // VGPRs of loads in flight per thread); adds stay in token order.
        constexpr int kBatch = 16 / (NK * (In::bytes / 2)) > 0 ? 16 / (NK * (In::bytes / 2)) : 1;
        cnt = kLeaf;
#pragma unroll
        for (int i0 = 0; i0 < kLeaf; i0 += kBatch) {
          Raw8<In> raw[kBatch][NK];
#pragma unroll
          for (int u = 0; u < kBatch; ++u)
#pragma unroll
            for (int k = 0; k < NK; ++k) raw[u][k] = ld8<In>(row[k] + (t0 + i0 + u) * step[k]);
#pragma unroll
          for (int u = 0; u < kBatch; ++u)
#pragma unroll
            for (int k = 0; k < NK; ++k) add8<In>(raw[u][k], acc[k]);
        }
      } else {
        for (int64_t t = t0; t < t1; ++t) {
          if (valid && !valid[t]) continue;
          ++cnt;
#pragma unroll
          for (int k = 0; k < NK; ++k) add8<In>(ld8<In>(row[k] + t * step[k]), acc[k]);
        }
      }
      float* out = table + (int64_t)e * W;
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        float4* o = reinterpret_cast<float4*>(out + 8 * (gl + 16 * k));
        o[0] = make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
        o[1] = make_float4(acc[k][4], acc[k][5], acc[k][6], acc[k][7]);
      }
      if (counts && gl == 0) pp.pcnt[(int64_t)b * pp.E + e] = cnt;
    } else {
      const float* row = table + (int64_t)(pp.off[base] + e) * W;
#pragma unroll
      for (int k = 0; k < NK; ++k) add_f8(row + 8 * (gl + 16 * k), acc[k]);
      if (counts) cnt = pp.pcnt[(int64_t)b * pp.E + pp.off[base] + e];
    }
  }
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int q = 0; q < 8; ++q) buf[0][r * W + 8 * (gl + 16 * k) + q] = acc[k][q];
  if (gl == 0) cbuf[0][r] = cnt;
  __syncthreads();
  for (int f = 1; f <= kFold; ++f) {
    const int L = base + f;
    if (L >= pp.levels) break;                      // uniform
    const float* in = buf[(f - 1) & 1];
    float* out = buf[f & 1];
    const int m = 16 >> f;
    const int first = seg * m;
    float* dst = table + (int64_t)(pp.off[L] + first) * W;
    for (int idx = threadIdx.x; idx < m * W; idx += kSumThreads) {
      const int i = idx / W, col = idx - i * W;
      const float v = in[2 * i * W + col] + in[(2 * i + 1) * W + col];
      out[idx] = v;
      if (first + i < pp.n[L]) dst[idx] = v;
    }
    if (counts && (int)threadIdx.x < m) {
      const int c = cbuf[(f - 1) & 1][2 * threadIdx.x] + cbuf[(f - 1) & 1][2 * threadIdx.x + 1];
      cbuf[f & 1][threadIdx.x] = c;
      if (first + (int)threadIdx.x < pp.n[L]) pp.pcnt[(int64_t)b * pp.E + pp.off[L] + first + threadIdx.x] = c;
    }
    __syncthreads();
  }
}

// The levels above `base` when level `base` holds at most kTopMax entries per
// (b, h): one workgroup per (b, h, chunk of kTopCols table columns) loads the
// chunk of every level-`base` entry into LDS and forms all higher levels there
// (entry i of a level = entries 2i and 2i+1 below, a missing right neighbour
// counted as 0, as in pyramid_kernel), writing each level to the table.
constexpr int kTopMax = 256, kTopCols = 8;
__global__ __launch_bounds__(kSumThreads) void pyramid_top_kernel(PyrParams pp, int base) {
  __shared__ float buf[2][kTopMax * kTopCols];
  __shared__ int cbuf[2][kTopMax];
  const SumParams& p = pp.p;
  const int W = 2 * p.D;
  const int nchunk = W / kTopCols;
  const int chunk = blockIdx.x % nchunk;
  const int bh = blockIdx.x / nchunk;
  const int b = bh / p.H, h = bh % p.H;
  const bool counts = pp.pcnt != nullptr && h == 0 && chunk == 0;
  float* table = pp.pyr + (int64_t)bh * pp.E * W + chunk * kTopCols;
  int n = pp.n[base];
  for (int idx = threadIdx.x; idx < n * kTopCols / 4; idx += kSumThreads) {
    const int i = idx / (kTopCols / 4), c4 = idx % (kTopCols / 4);
    reinterpret_cast<float4*>(buf[0])[idx] =
        reinterpret_cast<const float4*>(table + (int64_t)(pp.off[base] + i) * W)[c4];
  }
  if (counts)
    for (int i = threadIdx.x; i < n; i += kSumThreads) cbuf[0][i] = pp.pcnt[(int64_t)b * pp.E + pp.off[base] + i];
  __syncthreads();
  int cur = 0;
  for (int L = base + 1; L < pp.levels; ++L) {
    const int m = pp.n[L];
    const float* in = buf[cur];
    float* out = buf[cur ^ 1];
    float* dst = table + (int64_t)pp.off[L] * W;
    for (int idx = threadIdx.x; idx < m * kTopCols; idx += kSumThreads) {
      const int i = idx / kTopCols, col = idx % kTopCols;
      const float right = 2 * i + 1 < n ? in[(2 * i + 1) * kTopCols + col] : 0.f;
      const float v = in[2 * i * kTopCols + col] + right;
      out[idx] = v;
      dst[(int64_t)i * W + col] = v;
    }
    if (counts)
      for (int i = threadIdx.x; i < m; i += kSumThreads) {
        const int c = cbuf[cur][2 * i] + (2 * i + 1 < n ? cbuf[cur][2 * i + 1] : 0);
        cbuf[cur ^ 1][i] = c;
        pp.pcnt[(int64_t)b * pp.E + pp.off[L] + i] = c;
      }
    __syncthreads();
    cur ^= 1;
    n = m;
  }
}

// Four ranges per wavefront: 16-lane group grp = lane / 16 takes range item
// 4 * wave + grp (item = (b, h, range)), lane gl = lane % 16 its granule
// columns gl + 16k.  A group adds the partial leaves at the range ends and then
// the table entries covering the rest, in that order; a tree-node prototype
// range is a single entry.  No cross-lane traffic.
template <typename In, int NK>
__global__ __launch_bounds__(kSumThreads) void range_pyr_kernel(PyrParams pp) {
  const SumParams& p = pp.p;
  const int lane = threadIdx.x & 63;
  const int gl = lane & 15;
  const int64_t idx = ((int64_t)blockIdx.x * (kSumThreads / 64) + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  if (idx >= (int64_t)p.B * p.H * p.R) return;  // no barrier follows
  const int r = (int)(idx % p.R);
  const int bh = (int)(idx / p.R);
  const int h = bh % p.H, b = bh / p.H;
  // Ranges come from caller memory: clamp them to [0, T] so a bad table can
  // only produce wrong sums, never an out-of-bounds read.
  int64_t s = p.starts[r], e = p.ends[r];
  s = s < 0 ? 0 : (s > p.T ? p.T : s);
  e = e < s ? s : (e > p.T ? p.T : e);
  // Whole leaves [c0, c1); the last leaf may be short (tokens past T do not
  // exist), so a range ending at T takes it whole.
  const int64_t epad = e == p.T ? (int64_t)pp.n[0] * kLeaf : e;
  int64_t c0 = (s + kLeaf - 1) / kLeaf, c1 = epad / kLeaf;
  int64_t head_end = c0 * kLeaf, tail_start = c1 * kLeaf;
  if (c1 <= c0) {
    c0 = c1 = 0;
    head_end = e;
    tail_start = e;
  }
  const int nh = (int)(head_end - s), nt = (int)(e > tail_start ? e - tail_start : 0);
  const int W = 2 * p.D;
  float acc[NK][8];
#pragma unroll
  for (int k = 0; k < NK; ++k)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[k][q] = 0.f;
  const uint8_t* valid = p.valid ? p.valid + (int64_t)b * p.T : nullptr;
  int nvalid = 0;
  if (nh + nt > 0) {
    const char* row[NK];
    int64_t step[NK];
    granule_ptrs<In, NK>(p, b, h, gl, row, step);
    for (int i = 0; i < nh + nt; ++i) {
      const int64_t t = i < nh ? s + i : tail_start + (i - nh);
      if (valid && !valid[t]) continue;
      ++nvalid;
#pragma unroll
      for (int k = 0; k < NK; ++k) add8<In>(ld8<In>(row[k] + t * step[k]), acc[k]);
    }
  }
  const float* table = pp.pyr + (int64_t)bh * pp.E * W;
  for (int64_t c = c0; c < c1;) {
    // Largest aligned power-of-two block of leaves starting at c inside [c, c1).
    int j = 63 - __builtin_clzll((unsigned long long)(c1 - c));
    if (c != 0) {
      const int a = __builtin_ctzll((unsigned long long)c);
      j = a < j ? a : j;
    }
    const int64_t ent = pp.off[j] + (c >> j);
#pragma unroll
    for (int k = 0; k < NK; ++k) add_f8(table + ent * W + 8 * (gl + 16 * k), acc[k]);
    if (valid) nvalid += pp.pcnt[(int64_t)b * pp.E + ent];
    c += (int64_t)1 << j;
  }
  const int count = valid ? nvalid : (int)(e - s);
  const float denom = count > 1 ? (float)count : 1.0f;
  const int64_t orow = (((int64_t)b * p.H + h) * p.R + r) * p.D;
  const int G = p.D / 8;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int gc = gl + 16 * k;
    const int which = gc >= G, d0 = 8 * (which ? gc - G : gc);
    float4* o = reinterpret_cast<float4*>((which ? p.values : p.keys) + orow + d0);
    o[0] = make_float4(acc[k][0] / denom, acc[k][1] / denom, acc[k][2] / denom, acc[k][3] / denom);
    o[1] = make_float4(acc[k][4] / denom, acc[k][5] / denom, acc[k][6] / denom, acc[k][7] / denom);
  }
  if (h == 0 && gl == 0) {
    p.counts[(int64_t)b * p.R + r] = (float)count;
    p.log_counts[(int64_t)b * p.R + r] = count > 0 ? logf((float)count) : -__builtin_inff();
  }
}

template <typename In, int NK>
int launch_dyadic(const PyrParams& pp, int64_t g2, hipStream_t stream) {
  const size_t lds = (size_t)(24 * 2 * pp.p.D) * sizeof(float) + 32 * sizeof(int);
  for (int src = -1; src < pp.levels - 1; src = src < 0 ? kFold : src + kFold) {
    const int64_t nb = pp.n[src < 0 ? 0 : src];
    if (src >= 0 && nb <= kTopMax && (2 * pp.p.D) % kTopCols == 0) {
      // Every level above src in one launch.
      const int64_t grid = (int64_t)pp.p.B * pp.p.H * (2 * pp.p.D / kTopCols);
      hipLaunchKernelGGL(pyramid_top_kernel, dim3((unsigned)grid), dim3(kSumThreads), 0, stream, pp, src);
      const int rc = check_launch("pyramid_top_kernel");
      if (rc) return rc;
      break;
    }
    const int64_t grid = (int64_t)pp.p.B * pp.p.H * ((nb + 15) / 16);
    hipLaunchKernelGGL((pyramid_kernel<In, NK>), dim3((unsigned)grid), dim3(kSumThreads), lds, stream, pp, src);
    const int rc = check_launch("pyramid_kernel");
    if (rc) return rc;
  }
  const int64_t g3 = (g2 + kSumThreads / 16 - 1) / (kSumThreads / 16);
  hipLaunchKernelGGL((range_pyr_kernel<In, NK>), dim3((unsigned)g3), dim3(kSumThreads), 0, stream, pp);
  return check_launch("range_pyr_kernel");
}

template <typename In>
int launch_dyadic_nk(const PyrParams& pp, int64_t g2, hipStream_t stream) {
  switch (pp.p.D / 64) {
    case 1: return launch_dyadic<In, 1>(pp, g2, stream);
    case 2: return launch_dyadic<In, 2>(pp, g2, stream);
    case 3: return launch_dyadic<In, 3>(pp, g2, stream);
    default: return launch_dyadic<In, 4>(pp, g2, stream);
  }
}

size_t workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D) {
  auto up = [](size_t x) { return ((x + 255) / 256) * 256; };
  const int64_t nchunks = (T + kChunk - 1) / kChunk;
  const size_t scalar = up((size_t)(B * H * nchunks * 2 * D) * sizeof(float)) + (size_t)(B * nchunks) * sizeof(int);
  int64_t E = 0;
  table_levels(T, nullptr, nullptr, &E);
  const size_t dyadic = up((size_t)(B * H * E * 2 * D) * sizeof(float)) + (size_t)(B * E) * sizeof(int);
  return scalar > dyadic ? scalar : dyadic;
}

}  // namespace
}  // namespace spruce

using namespace spruce;

extern "C" size_t spruce_kv_summary_workspace_bytes(int64_t B, int64_t Hkv, int64_t T, int64_t D) {
  if (B < 1 || Hkv < 1 || T < 1 || D < 1) return 0;
  return workspace_bytes(B, Hkv, T, D);
}

namespace spruce {
namespace {

// The body of spruce_kv_summary and spruce_kv_summary_noalloc: `workspace`
// is caller memory or the library's static scratch.  Every workspace entry
// is written by the first launches before any launch reads it, so it needs
// no clearing between calls.
int kv_summary_run(const void* k, const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B, int64_t Hkv,
                   int64_t T, int64_t D, int dtype, const uint8_t* valid, const int64_t* range_starts,
                   const int64_t* range_ends, int64_t R, float* keys, float* values, float* counts,
                   float* log_counts, void* workspace, size_t workspace_bytes_given, void* stream) {
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
  char* ws = static_cast<char*>(workspace);
  p.chunk = reinterpret_cast<float*>(ws);
  p.chunk_cnt = reinterpret_cast<int*>(ws + up(sums));
  p.keys = keys; p.values = values; p.counts = counts; p.log_counts = log_counts;
  const int64_t g1 = B * Hkv * (int64_t)p.nchunks, g2 = B * Hkv * R;
  SPRUCE_REQUIRE(g1 < ((int64_t)1 << 31) && g2 < ((int64_t)1 << 31), "too many workgroups");
  const int eb = dtype == SPRUCE_DTYPE_F32 ? 4 : 2;
  const bool vec = D % 64 == 0 && D <= 256 && ks[3] == 1 && vs[3] == 1 && ((uintptr_t)k % 16) == 0 &&
                   ((uintptr_t)v % 16) == 0 && ((uintptr_t)keys % 16) == 0 && ((uintptr_t)values % 16) == 0 &&
                   (ks[0] * eb) % 16 == 0 && (ks[1] * eb) % 16 == 0 &&
                   (ks[2] * eb) % 16 == 0 && (vs[0] * eb) % 16 == 0 && (vs[1] * eb) % 16 == 0 &&
                   (vs[2] * eb) % 16 == 0;
  if (!vec) {
    hipLaunchKernelGGL(chunk_sum_kernel, dim3((unsigned)g1), dim3(kSumThreads), 0, (hipStream_t)stream, p);
    int rc = check_launch("chunk_sum_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(range_sum_kernel, dim3((unsigned)g2), dim3(kSumThreads), 0, (hipStream_t)stream, p);
    return check_launch("range_sum_kernel");
  }
  PyrParams pp;
  pp.p = p;
  int64_t n[64], off[64], E = 0;
  pp.levels = table_levels(T, n, off, &E);
  SPRUCE_REQUIRE(pp.levels <= kMaxLevels, "sequence too long");
  for (int i = 0; i < pp.levels; ++i) { pp.n[i] = (int)n[i]; pp.off[i] = (int)off[i]; }
  pp.E = (int)E;
  pp.pyr = reinterpret_cast<float*>(ws);
  pp.pcnt = valid ? reinterpret_cast<int*>(ws + up((size_t)(B * Hkv * E * 2 * D) * sizeof(float))) : nullptr;
  if (dtype == SPRUCE_DTYPE_BF16) return launch_dyadic_nk<InBF16>(pp, g2, (hipStream_t)stream);
  if (dtype == SPRUCE_DTYPE_F16) return launch_dyadic_nk<InF16>(pp, g2, (hipStream_t)stream);
  return launch_dyadic_nk<InF32>(pp, g2, (hipStream_t)stream);
}

}  // namespace
}  // namespace spruce

extern "C" int spruce_kv_summary(const void* k, const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B,
                                 int64_t Hkv, int64_t T, int64_t D, int dtype, const uint8_t* valid,
                                 const int64_t* range_starts, const int64_t* range_ends, int64_t R, float* keys,
                                 float* values, float* counts, float* log_counts, void* workspace,
                                 size_t workspace_bytes_given, void* stream) {
  return kv_summary_run(k, ks, v, vs, B, Hkv, T, D, dtype, valid, range_starts, range_ends, R, keys, values, counts,
                        log_counts, workspace, workspace_bytes_given, stream);
}

// ------------------------------------------------------- allocation-free form
// The workspace of spruce_kv_summary_noalloc: one copy per GPU, created when
// the library's code object is loaded on that GPU and held until the process
// ends.  Host code never uses this name as an address (on the host it is a
// stand-in symbol): the device address comes from hipGetSymbolAddress, looked
// up once per device with that device current.
static __device__ __align__(256) unsigned char scratch[SPRUCE_KV_SUMMARY_NOALLOC_MAX_BYTES];

namespace {

constexpr int kMaxDevices = 64;
// Guards the per-device tables below, and is held by a call from its ordering
// wait to its ordering record, so calls from several host threads enter one at
// a time.
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
// Recorded after each call's launches; the next call on the device makes its
// stream wait for it, so calls on different streams do not share the scratch
// at the same time.
hipEvent_t g_scratch_done[kMaxDevices] = {};

// Device address of `scratch` on the current device and that device's
// ordering event, set up on the device's first call.  The current device must
// be the device of `stream` (a stream of another device would run the kernels
// where this address is not mapped).  The caller holds g_scratch_mu.
int scratch_for_stream(void* stream, void** out, hipEvent_t* done) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return spruce::set_error((int)e, "hipGetDevice failed: %s", hipGetErrorString(e));
  SPRUCE_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d outside the %d devices supported", dev, kMaxDevices);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return spruce::set_error((int)e, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
    SPRUCE_REQUIRE(sdev == dev, "stream belongs to device %d but device %d is current", (int)sdev, dev);
  }
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return spruce::set_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol,
                               "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess)
      return spruce::set_error((int)e, "hipEventCreateWithFlags failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  *done = g_scratch_done[dev];
  return 0;
}

}  // namespace

extern "C" int spruce_kv_summary_noalloc(const void* k, const int64_t ks[4], const void* v, const int64_t vs[4],
                                         int64_t B, int64_t Hkv, int64_t T, int64_t D, int dtype,
                                         const uint8_t* valid, const int64_t* range_starts,
                                         const int64_t* range_ends, int64_t R, float* keys, float* values,
                                         float* counts, float* log_counts, void* stream) {
  SPRUCE_REQUIRE(B >= 1 && Hkv >= 1 && T >= 1 && D >= 1, "invalid shape");
  SPRUCE_REQUIRE(B < (1 << 20) && Hkv < (1 << 16) && T < ((int64_t)1 << 30) && D <= 4096, "shape out of range");
  const size_t need = workspace_bytes(B, Hkv, T, D);
  SPRUCE_REQUIRE(need <= (size_t)SPRUCE_KV_SUMMARY_NOALLOC_MAX_BYTES,
                 "spruce_kv_summary_noalloc: this shape needs %zu bytes of scratch, above its limit of %zu bytes "
                 "(use spruce_kv_summary with a caller workspace)",
                 need, (size_t)SPRUCE_KV_SUMMARY_NOALLOC_MAX_BYTES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  void* ws = nullptr;
  hipEvent_t done = nullptr;
  int rc = scratch_for_stream(stream, &ws, &done);
  if (rc) return rc;
  // Under stream capture the event would tie the graph to work outside it:
  // a captured call is ordered by the caller's graph alone.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing((hipStream_t)stream, &capture);
  if (e != hipSuccess) return spruce::set_error((int)e, "hipStreamIsCapturing failed: %s", hipGetErrorString(e));
  const bool ordered = capture == hipStreamCaptureStatusNone;
  if (ordered) {
    // The previous call's kernels on this device (any stream) finish first;
    // before the first record the wait is already satisfied.
    e = hipStreamWaitEvent((hipStream_t)stream, done, 0);
    if (e != hipSuccess) return spruce::set_error((int)e, "hipStreamWaitEvent failed: %s", hipGetErrorString(e));
  }
  rc = kv_summary_run(k, ks, v, vs, B, Hkv, T, D, dtype, valid, range_starts, range_ends, R, keys, values, counts,
                      log_counts, ws, (size_t)SPRUCE_KV_SUMMARY_NOALLOC_MAX_BYTES, stream);
  if (ordered) {
    // Recorded whatever rc is: a failed call may have launched some kernels.
    e = hipEventRecord(done, (hipStream_t)stream);
    if (e != hipSuccess && rc == 0)
      return spruce::set_error((int)e, "hipEventRecord failed: %s", hipGetErrorString(e));
  }
  return rc;
}
