// Selector front end on gfx950: block pooling, gate projection, MaxSim block
// scores and causal top-k block selection.
//
// Selected block indices are compared bit for bit with a CPU restatement, so
// every floating-point value is produced by a fixed sequence of IEEE single
// operations (this file is built with -ffp-contract=off; fused multiply-adds
// appear only where __builtin_fmaf is written, divisions are IEEE):
//   pool    per token the G query heads are summed left to right; token t of a
//           64-token block belongs to lane t % L (L = the largest power of two
//           <= min(64, 256 / (D/8)), so L lanes of 64 / L tokens cover the
//           block exactly and the halving tree reaches every lane);
//           a lane folds its tokens in increasing order starting from the first
//           token's value; lanes combine by a halving tree; the sum is divided
//           by G * (real tokens).  Missing tokens add +0.0f to sums, nothing to
//           maxima.  (teacher/chunked_extract.py:75-80 group average,
//           :27-72 prototype 0 block mean; plus the per-dim block max.)
//   project fmaf chain over the input dim, from 0 (selector/gate.py:120-127).
//   scores  max over prototype pairs (query prototype major, first pair taken
//           as is, later pairs replace it only when strictly larger) of fmaf
//           chains over the projection dim, divided by sqrt(p)
//           (selector/gate.py:29-101); above the diagonal -inf
//           (selector/recall.py:26-35).
//   top-k   per row the k largest causal scores, ties to the lower block index
//           (stable descending argsort, selector/baselines.py:59-62), written
//           ascending with -1 padding (interfaces/selected_blocks_spec.md).
//
// The pooling kernel streams Q and K once from HBM (the dominant cost of the
// front end: Q is 7x the bytes of K at 28/4 heads); the rest touches only the
// pooled summaries and the [Qb, Kb] score matrix.
#include "common.h"

namespace spruce {

constexpr int kSelBlock = 64;

// Token lanes per 8-dim chunk of the pooling kernels: the largest power of two
// with lanes * (D / 8) <= 256 threads, at most one lane per token of a block.
__host__ __device__ constexpr int pool_lanes(int dch) {
  int lanes = kSelBlock;
  while (lanes > 1 && lanes * dch > 256) lanes /= 2;
  return lanes;
}

struct PoolParams {
  const void* q;
  const void* k;
  int64_t qs[4], ks[4];
  int B, Hq, Hkv, T, D, G, nb, dtype;
  float* q_mean;  // [B, Hkv, nb, D]
  float* k_sum;   // [B, Hkv, nb, 2, D] (mean, max)
};

// Total order on floats as unsigned keys (+0 above -0).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float max_total(float a, float b) { return order_key(b) > order_key(a) ? b : a; }

// One workgroup per (batch, KV head, 64-token block); thread = (token lane l,
// dim chunk c of 8 dims).
__global__ __launch_bounds__(256) void block_pool_kernel(const PoolParams p) {
  __shared__ float red[256 * 8];
  __shared__ float redmax[256 * 8];
  const int dch = p.D / 8;
  const int L = pool_lanes(dch);
  const int per = kSelBlock / L;
  const int tid = threadIdx.x;
  const int l = tid / dch, c = tid - (tid / dch) * dch;
  int w = blockIdx.x;
  const int blk = w % p.nb;
  w /= p.nb;
  const int g = w % p.Hkv;
  const int b = w / p.Hkv;
  const int t0 = blk * kSelBlock;
  int n = p.T - t0;
  n = n > kSelBlock ? kSelBlock : n;
  const bool work = tid < dch * L;

  if (p.q) {
    float acc[8];
    if (work) {
      for (int i = 0; i < per; ++i) {
        const int t = t0 + l + i * L;
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (t < p.T) {
          load8f(p.q, (int64_t)b * p.qs[0] + (int64_t)(g * p.G) * p.qs[1] + (int64_t)t * p.qs[2] + 8 * c, p.dtype, s);
          for (int h = 1; h < p.G; ++h) {
            float x[8];
            load8f(p.q, (int64_t)b * p.qs[0] + (int64_t)(g * p.G + h) * p.qs[1] + (int64_t)t * p.qs[2] + 8 * c,
                   p.dtype, x);
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] = s[e] + x[e];
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = (i == 0) ? s[e] : acc[e] + s[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) red[(l * dch + c) * 8 + e] = acc[e];
    }
    __syncthreads();
    for (int st = L / 2; st >= 1; st /= 2) {
      if (work && l < st) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          red[(l * dch + c) * 8 + e] = red[(l * dch + c) * 8 + e] + red[((l + st) * dch + c) * 8 + e];
      }
      __syncthreads();
    }
    if (work && l == 0) {
      const float den = (float)(p.G * n);
      float* o = p.q_mean + (((int64_t)b * p.Hkv + g) * p.nb + blk) * p.D + 8 * c;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = red[c * 8 + e] / den;
    }
    __syncthreads();
  }

  if (p.k) {
    float acc[8], mx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mx[e] = -INFINITY;
    if (work) {
      for (int i = 0; i < per; ++i) {
        const int t = t0 + l + i * L;
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (t < p.T) {
          load8f(p.k, (int64_t)b * p.ks[0] + (int64_t)g * p.ks[1] + (int64_t)t * p.ks[2] + 8 * c, p.dtype, s);
#pragma unroll
          for (int e = 0; e < 8; ++e) mx[e] = max_total(mx[e], s[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = (i == 0) ? s[e] : acc[e] + s[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        red[(l * dch + c) * 8 + e] = acc[e];
        redmax[(l * dch + c) * 8 + e] = mx[e];
      }
    }
    __syncthreads();
    for (int st = L / 2; st >= 1; st /= 2) {
      if (work && l < st) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          red[(l * dch + c) * 8 + e] = red[(l * dch + c) * 8 + e] + red[((l + st) * dch + c) * 8 + e];
          redmax[(l * dch + c) * 8 + e] = max_total(redmax[(l * dch + c) * 8 + e], redmax[((l + st) * dch + c) * 8 + e]);
        }
      }
      __syncthreads();
    }
    if (work && l == 0) {
      const float den = (float)n;
      float* o = p.k_sum + ((((int64_t)b * p.Hkv + g) * p.nb + blk) * 2) * p.D + 8 * c;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] = red[c * 8 + e] / den;
        o[p.D + e] = redmax[c * 8 + e];
      }
    }
  }
}

// 8 consecutive elements of TIn as raw bits, widened after the load returns.
template <typename TIn>
struct Raw8 {
  uint4 a;
};
template <>
struct Raw8<InF32> {
  float4 a, b;
};

template <typename TIn>
__device__ __forceinline__ Raw8<TIn> raw8_at(const void* base, int64_t elem) {
  Raw8<TIn> r;
  if constexpr (TIn::bytes == 4) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    r.a = q[0];
    r.b = q[1];
  } else {
    r.a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
  }
  return r;
}

template <typename TIn>
__device__ __forceinline__ void widen8(const Raw8<TIn>& r, float* out) {
  if constexpr (TIn::bytes == 4) {
    out[0] = r.a.x; out[1] = r.a.y; out[2] = r.a.z; out[3] = r.a.w;
    out[4] = r.b.x; out[5] = r.b.y; out[6] = r.b.z; out[7] = r.b.w;
  } else {
    constexpr bool F16 = TIn::code == SPRUCE_DTYPE_F16;
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = unpack1<F16>(w[i] & 0xffffu);
      out[2 * i + 1] = unpack1<F16>(w[i] >> 16);
    }
  }
}

// block_pool_kernel with every load issued ahead of its use: the input type
// is a template parameter (no per-load dtype branch), the G heads of a token
// step are loaded together (G <= kPoolMaxG), and the K rows of the thread's
// token steps (at most kPoolMaxPer) are loaded before the Q part starts.
// Identical arithmetic: per token the heads summed left to right, token steps
// folded in order, the same halving tree, the same divisions.
constexpr int kPoolMaxG = 8, kPoolMaxPer = 8;
template <typename TIn>
__global__ __launch_bounds__(256) void block_pool_fast_kernel(const PoolParams p) {
  __shared__ float red[256 * 8];
  __shared__ float redmax[256 * 8];
  const int dch = p.D / 8;
  const int L = pool_lanes(dch);
  const int per = kSelBlock / L;
  const int tid = threadIdx.x;
  const int l = tid / dch, c = tid - (tid / dch) * dch;
  int w = blockIdx.x;
  const int blk = w % p.nb;
  w /= p.nb;
  const int g = w % p.Hkv;
  const int b = w / p.Hkv;
  const int t0 = blk * kSelBlock;
  int n = p.T - t0;
  n = n > kSelBlock ? kSelBlock : n;
  const bool work = tid < dch * L;

  Raw8<TIn> kr[kPoolMaxPer];
  if (p.k && work) {
#pragma unroll
    for (int i = 0; i < kPoolMaxPer; ++i) {
      const int t = t0 + l + i * L;
      if (i < per && t < p.T)
        kr[i] = raw8_at<TIn>(p.k, (int64_t)b * p.ks[0] + (int64_t)g * p.ks[1] + (int64_t)t * p.ks[2] + 8 * c);
    }
  }

  if (p.q) {
    float acc[8];
    if (work) {
      for (int i = 0; i < per; ++i) {
        const int t = t0 + l + i * L;
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (t < p.T) {
          const int64_t e0 = (int64_t)b * p.qs[0] + (int64_t)(g * p.G) * p.qs[1] + (int64_t)t * p.qs[2] + 8 * c;
          Raw8<TIn> qr[kPoolMaxG];
#pragma unroll
          for (int h = 0; h < kPoolMaxG; ++h)
            if (h < p.G) qr[h] = raw8_at<TIn>(p.q, e0 + (int64_t)h * p.qs[1]);
          widen8<TIn>(qr[0], s);
#pragma unroll
          for (int h = 1; h < kPoolMaxG; ++h) {
            if (h < p.G) {
              float x[8];
              widen8<TIn>(qr[h], x);
#pragma unroll
              for (int e = 0; e < 8; ++e) s[e] = s[e] + x[e];
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = (i == 0) ? s[e] : acc[e] + s[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) red[(l * dch + c) * 8 + e] = acc[e];
    }
    __syncthreads();
    for (int st = L / 2; st >= 1; st /= 2) {
      if (work && l < st) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          red[(l * dch + c) * 8 + e] = red[(l * dch + c) * 8 + e] + red[((l + st) * dch + c) * 8 + e];
      }
      __syncthreads();
    }
    if (work && l == 0) {
      const float den = (float)(p.G * n);
      float* o = p.q_mean + (((int64_t)b * p.Hkv + g) * p.nb + blk) * p.D + 8 * c;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = red[c * 8 + e] / den;
    }
    __syncthreads();
  }

  if (p.k) {
    float acc[8], mx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mx[e] = -INFINITY;
    if (work) {
#pragma unroll
      for (int i = 0; i < kPoolMaxPer; ++i) {
        if (i >= per) break;
        const int t = t0 + l + i * L;
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (t < p.T) {
          widen8<TIn>(kr[i], s);
#pragma unroll
          for (int e = 0; e < 8; ++e) mx[e] = max_total(mx[e], s[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = (i == 0) ? s[e] : acc[e] + s[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        red[(l * dch + c) * 8 + e] = acc[e];
        redmax[(l * dch + c) * 8 + e] = mx[e];
      }
    }
    __syncthreads();
    for (int st = L / 2; st >= 1; st /= 2) {
      if (work && l < st) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          red[(l * dch + c) * 8 + e] = red[(l * dch + c) * 8 + e] + red[((l + st) * dch + c) * 8 + e];
          redmax[(l * dch + c) * 8 + e] = max_total(redmax[(l * dch + c) * 8 + e], redmax[((l + st) * dch + c) * 8 + e]);
        }
      }
      __syncthreads();
    }
    if (work && l == 0) {
      const float den = (float)n;
      float* o = p.k_sum + ((((int64_t)b * p.Hkv + g) * p.nb + blk) * 2) * p.D + 8 * c;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] = red[c * 8 + e] / den;
        o[p.D + e] = redmax[c * 8 + e];
      }
    }
  }
}

// out[n][j] = fmaf chain over d (in order, from 0) of x[n][d] * w[d][j].
// A workgroup computes a 32 x 64 output tile, each thread a 2 x 4 register
// tile; x and w are staged through LDS in 128-wide slices of d (one slice for
// head_dim <= 128), so there is one load round trip per slice.
constexpr int kPR = 32, kPC = 64, kPD = 128;
__global__ __launch_bounds__(256) void project_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      int64_t N, int D, int P, float* __restrict__ out) {
  __shared__ float xs[kPR][kPD + 1];
  __shared__ __attribute__((aligned(16))) float ws[kPD][kPC];
  const int tid = threadIdx.x;
  const int tr = tid >> 4, tc = tid & 15;
  const int64_t n0 = (int64_t)blockIdx.x * kPR;
  const int j0 = blockIdx.y * kPC;
  float acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[a][c] = 0.f;
  for (int d0 = 0; d0 < D; d0 += kPD) {
    const int dn = D - d0 < kPD ? D - d0 : kPD;
    // All loads of the slice are issued before any LDS store (one round trip).
    float xv_[kPR * kPD / 256], wv_[kPD * kPC / 256];
#pragma unroll
    for (int t = 0; t < kPR * kPD / 256; ++t) {
      const int e = tid + 256 * t, r = e / kPD, dd = e % kPD;
      const int64_t n = n0 + r;
      xv_[t] = (n < N && dd < dn) ? x[n * D + d0 + dd] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < kPD * kPC / 256; ++t) {
      const int e = tid + 256 * t, dd = e / kPC, jj = e % kPC;
      wv_[t] = (dd < dn && j0 + jj < P) ? w[(int64_t)(d0 + dd) * P + j0 + jj] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < kPR * kPD / 256; ++t) {
      const int e = tid + 256 * t;
      xs[e / kPD][e % kPD] = xv_[t];
    }
#pragma unroll
    for (int t = 0; t < kPD * kPC / 256; ++t) {
      const int e = tid + 256 * t;
      ws[e / kPC][e % kPC] = wv_[t];
    }
    __syncthreads();
#pragma unroll 8
    for (int dd = 0; dd < dn; ++dd) {
      const float4 wv = *reinterpret_cast<const float4*>(&ws[dd][4 * tc]);
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const float xv = xs[2 * tr + a][dd];
        acc[a][0] = __builtin_fmaf(xv, wv.x, acc[a][0]);
        acc[a][1] = __builtin_fmaf(xv, wv.y, acc[a][1]);
        acc[a][2] = __builtin_fmaf(xv, wv.z, acc[a][2]);
        acc[a][3] = __builtin_fmaf(xv, wv.w, acc[a][3]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int64_t n = n0 + 2 * tr + a;
    if (n >= N) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j = j0 + 4 * tc + c;
      if (j < P) out[n * P + j] = acc[a][c];
    }
  }
}

// Vector form for D % 4 == 0, P % 4 == 0 and 16-byte aligned operands: a
// 16TR x 64 output tile per workgroup, a TR x 4 register tile per thread, x
// staged transposed so every step reads TR floats of x and one float4 of w
// from LDS for 4TR FMAs (the scalar form above reads 3 values for 8).  Same
// fmaf chain per output (d in order from 0), so the results are identical.
// One launch can carry two projections (the query and key prototypes of the
// selector): row tiles [0, tiles_a) belong to problem a, the rest to b.
constexpr int kVC = 64, kVD = 128;
struct ProjPair {
  const float* xa;
  const float* wa;
  float* outa;
  const float* xb;
  const float* wb;
  float* outb;
  int64_t na, nb, tiles_a;
  int D, P;
};

template <int TR>
__global__ __launch_bounds__(256) void project_tile_kernel(const ProjPair pp) {
  constexpr int R = 16 * TR;   // rows per tile
  constexpr int XL = R / 8;    // float4 of x per thread per slice
  __shared__ __attribute__((aligned(16))) float xs[kVD][R + 4];
  __shared__ __attribute__((aligned(16))) float ws[kVD][kVC];
  const bool second = (int64_t)blockIdx.x >= pp.tiles_a;
  const float* __restrict__ x = second ? pp.xb : pp.xa;
  const float* __restrict__ w = second ? pp.wb : pp.wa;
  float* __restrict__ out = second ? pp.outb : pp.outa;
  const int64_t N = second ? pp.nb : pp.na;
  const int D = pp.D, P = pp.P;
  const int tid = threadIdx.x;
  const int tr = tid >> 4, tc = tid & 15;
  const int64_t n0 = ((int64_t)blockIdx.x - (second ? pp.tiles_a : 0)) * R;
  const int j0 = blockIdx.y * kVC;
  float acc[TR][4];
#pragma unroll
  for (int a = 0; a < TR; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[a][c] = 0.f;
  for (int d0 = 0; d0 < D; d0 += kVD) {
    const int dn = D - d0 < kVD ? D - d0 : kVD;
    float4 xv[XL], wv[8];
    // x is staged row-fastest (lane r of a wave reads row r's float4), so the
    // transposed LDS stores of a wave fall in distinct banks.
#pragma unroll
    for (int t = 0; t < XL; ++t) {
      const int e = tid + 256 * t, r = e % R, c4 = e / R;
      const int64_t n = n0 + r;
      xv[t] = (n < N && 4 * c4 < dn) ? *reinterpret_cast<const float4*>(x + n * D + d0 + 4 * c4)
                                     : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int e = tid + 256 * t, dd = e >> 4, c4 = e & 15;
      const int j = j0 + 4 * c4;
      wv[t] = (dd < dn && j < P) ? *reinterpret_cast<const float4*>(w + (int64_t)(d0 + dd) * P + j)
                                 : float4{0.f, 0.f, 0.f, 0.f};
    }
    if (d0 > 0) __syncthreads();  // the previous slice's reads are done
#pragma unroll
    for (int t = 0; t < XL; ++t) {
      const int e = tid + 256 * t, r = e % R, c4 = e / R;
      xs[4 * c4][r] = xv[t].x;
      xs[4 * c4 + 1][r] = xv[t].y;
      xs[4 * c4 + 2][r] = xv[t].z;
      xs[4 * c4 + 3][r] = xv[t].w;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int e = tid + 256 * t, dd = e >> 4, c4 = e & 15;
      *reinterpret_cast<float4*>(&ws[dd][4 * c4]) = wv[t];
    }
    __syncthreads();
#pragma unroll 4
    for (int dd = 0; dd < dn; ++dd) {
      float av[TR];
#pragma unroll
      for (int a = 0; a < TR; a += 2) {
        const float2 a2 = *reinterpret_cast<const float2*>(&xs[dd][TR * tr + a]);
        av[a] = a2.x;
        av[a + 1] = a2.y;
      }
      const float4 b4 = *reinterpret_cast<const float4*>(&ws[dd][4 * tc]);
      const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int a = 0; a < TR; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = __builtin_fmaf(av[a], bv[c], acc[a][c]);
    }
  }
  const int j = j0 + 4 * tc;
  if (j >= P) return;
#pragma unroll
  for (int a = 0; a < TR; ++a) {
    const int64_t n = n0 + TR * tr + a;
    if (n < N) *reinterpret_cast<float4*>(out + n * P + j) = float4{acc[a][0], acc[a][1], acc[a][2], acc[a][3]};
  }
}

// Large-N form of the kernel above: a TR x TC register tile per thread
// (16 x 16 threads, a 16TR x 16TC output tile per workgroup) and d staged in
// slices of kBD, so each step reads TR / 4 + TC / 4 float4 from LDS for
// TR * TC FMAs (8 x 4: 96 bytes per FMA instruction against 128 for 4 x 4,
// whose reads alone keep the LDS busy). Same fmaf chain per output (d in
// order from 0), so the results are identical. Requires D % 4 == 0,
// P % 4 == 0 and 16-byte aligned operands.
constexpr int kBD = 32;
// 8 x 4 per thread from 16K rows (fewer rows leave CUs idle with 128-row
// tiles). Measured at p = d = 128: N = 131072 0.102 -> 0.068 ms, N = 65536
// 0.056 -> 0.039 ms; 8 x 8 and 4 x 8 within 5% of 8 x 4.
constexpr int kBlockProjectRows = 16384, kBlockProjectTR = 8, kBlockProjectTC = 4;

// Input rows of project_block_kernel: row n of one contiguous float32 [N, D]
// buffer ...
struct ProjRowsF32 {
  const float* x;
  __device__ const void* row(int64_t n, int D) const { return x + n * D; }
};

// ... or of prototype buffers in the model dtype, one per tree level: output
// row ((s * N + node) * P + proto) reads level v's [S, n_v, P, D] buffer at
// node - off[v].  Each value is widened to float32 exactly, so the chains see
// the same operands as after a float32 copy.
constexpr int kProjMaxSeg = 32;
struct ProjSegs {
  const void* base[kProjMaxSeg];
  int64_t off[kProjMaxSeg + 1];  // level v holds nodes off[v] .. off[v + 1] - 1; off[nseg] = N
  int nseg, P;
  int64_t N;
};
template <typename TIn>
struct ProjRowsSeg {
  ProjSegs g;
  __device__ const void* row(int64_t n, int D) const {
    const int64_t np = g.N * g.P;
    const int64_t sl = n / np, rem = n - sl * np;
    const int64_t node = rem / g.P, proto = rem - node * g.P;
    int v = 0;
    while (v + 1 < g.nseg && node >= g.off[v + 1]) ++v;
    const int64_t nv = g.off[v + 1] - g.off[v];
    return static_cast<const char*>(g.base[v]) + ((sl * nv + node - g.off[v]) * g.P + proto) * D * TIn::bytes;
  }
};

// Four consecutive input values at element e of a row, widened to float32.
__device__ __forceinline__ float4 load4_row(const ProjRowsF32&, const void* row, int e) {
  return *reinterpret_cast<const float4*>(static_cast<const float*>(row) + e);
}
template <typename TIn>
__device__ __forceinline__ float4 load4_row(const ProjRowsSeg<TIn>&, const void* row, int e) {
  if constexpr (TIn::bytes == 4) {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(row) + e);
  } else {
    constexpr bool F16 = TIn::code == SPRUCE_DTYPE_F16;
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(row) + e);
    return float4{unpack1<F16>(w.x & 0xffffu), unpack1<F16>(w.x >> 16), unpack1<F16>(w.y & 0xffffu),
                  unpack1<F16>(w.y >> 16)};
  }
}

// IL: rows are (node, prototype) pairs with ilk prototypes per node, and out
// is [nodes, P/4, ilk, 4] (each node's prototypes interleaved by 4-column
// group) instead of [N, P]; the output tile goes through LDS so that
// neighbouring lanes store neighbouring 16-byte slots.
template <int TR, int TC, typename Rows, bool IL = false>
__global__ __launch_bounds__(256) void project_block_kernel(const Rows src, const float* __restrict__ w, int64_t N,
                                                            int D, int P, float* __restrict__ out, int ilk = 0) {
  constexpr int R = 16 * TR, C = 16 * TC;          // workgroup tile
  constexpr int XL = R * kBD / 4 / 256;            // x float4 per thread per slice
  constexpr int WL = C * kBD / 4 / 256;            // w float4 per thread per slice
  constexpr int kXs = kBD * (R + 4), kWs = kBD * C, kOut = IL ? R * (C + 4) : 0;
  __shared__ __attribute__((aligned(16))) float smem[kXs + kWs > kOut ? kXs + kWs : kOut];
  float (*xs)[R + 4] = reinterpret_cast<float (*)[R + 4]>(smem);
  float (*ws)[C] = reinterpret_cast<float (*)[C]>(smem + kXs);
  const int tid = threadIdx.x;
  const int tr = tid >> 4, tc = tid & 15;
  const int64_t n0 = (int64_t)blockIdx.x * R;
  const int j0 = blockIdx.y * C;
  float acc[TR][TC];
#pragma unroll
  for (int a = 0; a < TR; ++a)
#pragma unroll
    for (int c = 0; c < TC; ++c) acc[a][c] = 0.f;
  // The rows this thread stages are the same in every slice.
  const void* xrow[XL];
#pragma unroll
  for (int t = 0; t < XL; ++t) {
    const int64_t n = n0 + (tid + 256 * t) / (kBD / 4);
    xrow[t] = n < N ? src.row(n, D) : nullptr;
  }
  for (int d0 = 0; d0 < D; d0 += kBD) {
    const int dn = D - d0 < kBD ? D - d0 : kBD;
    float4 xv[XL], wv[WL];
#pragma unroll
    for (int t = 0; t < XL; ++t) {
      const int c4 = (tid + 256 * t) % (kBD / 4);
      xv[t] = (xrow[t] != nullptr && 4 * c4 < dn) ? load4_row(src, xrow[t], d0 + 4 * c4)
                                                   : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int t = 0; t < WL; ++t) {
      const int e = tid + 256 * t, dd = e / (C / 4), c4 = e % (C / 4);
      const int j = j0 + 4 * c4;
      wv[t] = (dd < dn && j < P) ? *reinterpret_cast<const float4*>(w + (int64_t)(d0 + dd) * P + j)
                                 : float4{0.f, 0.f, 0.f, 0.f};
    }
    if (d0 > 0) __syncthreads();  // the previous slice's reads are done
#pragma unroll
    for (int t = 0; t < XL; ++t) {
      const int e = tid + 256 * t, r = e / (kBD / 4), c4 = e % (kBD / 4);
      xs[4 * c4][r] = xv[t].x;
      xs[4 * c4 + 1][r] = xv[t].y;
      xs[4 * c4 + 2][r] = xv[t].z;
      xs[4 * c4 + 3][r] = xv[t].w;
    }
#pragma unroll
    for (int t = 0; t < WL; ++t) {
      const int e = tid + 256 * t, dd = e / (C / 4), c4 = e % (C / 4);
      *reinterpret_cast<float4*>(&ws[dd][4 * c4]) = wv[t];
    }
    __syncthreads();
#pragma unroll 2
    for (int dd = 0; dd < dn; ++dd) {
      float av[TR], bv[TC];
#pragma unroll
      for (int a = 0; a < TR; a += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(&xs[dd][TR * tr + a]);
        av[a] = a4.x;
        av[a + 1] = a4.y;
        av[a + 2] = a4.z;
        av[a + 3] = a4.w;
      }
#pragma unroll
      for (int c = 0; c < TC; c += 4) {
        const float4 b4 = *reinterpret_cast<const float4*>(&ws[dd][TC * tc + c]);
        bv[c] = b4.x;
        bv[c + 1] = b4.y;
        bv[c + 2] = b4.z;
        bv[c + 3] = b4.w;
      }
#pragma unroll
      for (int a = 0; a < TR; ++a)
#pragma unroll
        for (int c = 0; c < TC; ++c) acc[a][c] = __builtin_fmaf(av[a], bv[c], acc[a][c]);
    }
  }
  if constexpr (IL) {
    // Tile [R][C + 4] in LDS, then slot s = (group g, row) with the row
    // fastest: consecutive rows of a node are consecutive 16-byte slots of
    // out (value (n, j) at node * ilk * P + (j / 4) * 4 * ilk + proto * 4).
    constexpr int OS = C + 4;
    __syncthreads();  // every read of xs / ws is done
#pragma unroll
    for (int a = 0; a < TR; ++a)
#pragma unroll
      for (int c = 0; c < TC; c += 4)
        *reinterpret_cast<float4*>(&smem[(TR * tr + a) * OS + TC * tc + c]) =
            float4{acc[a][c], acc[a][c + 1], acc[a][c + 2], acc[a][c + 3]};
    __syncthreads();
    for (int sl = tid; sl < R * (C / 4); sl += 256) {
      const int row = sl % R, g = sl / R;
      const int64_t n = n0 + row;
      const int j = j0 + 4 * g;
      if (n >= N || j >= P) continue;
      const int64_t node = n / ilk;
      *reinterpret_cast<float4*>(out + node * ilk * P + (int64_t)(j / 4) * 4 * ilk + (n - node * ilk) * 4) =
          *reinterpret_cast<const float4*>(&smem[row * OS + 4 * g]);
    }
  } else {
#pragma unroll
    for (int a = 0; a < TR; ++a) {
      const int64_t n = n0 + TR * tr + a;
      if (n >= N) continue;
#pragma unroll
      for (int c = 0; c < TC; c += 4) {
        const int j = j0 + TC * tc + c;
        if (j < P)
          *reinterpret_cast<float4*>(out + n * P + j) = float4{acc[a][c], acc[a][c + 1], acc[a][c + 2], acc[a][c + 3]};
      }
    }
  }
}

// MaxSim scores over a tile of 16 query blocks x 64 key blocks: lane = key
// block, wave = 4 query blocks (their prototype rows are LDS broadcasts).
// Each score is the fmaf chain over e (in order, from 0) of q . k, maximised
// over prototype pairs (a outer, c inner, strict >), then divided by div.
constexpr int kTI = 16, kTJ = 64, kRowsPerWave = kTI / 4;
struct ScoreParams {
  const float* qp;  // [BG, Qb, Pq, P]
  const float* kp;  // [BG, Kb, Pk, P]
  float* scores;    // [BG, Qb, Kb]
  int Qb, Kb, Pq, Pk, P;
  float div;
  int causal;  // 1: j > i is -inf and not computed; 2 (Qb == Kb): j > i unspecified
};

// Copies n float4 from src to LDS dst (dst index = map(e)), 8 loads in flight
// per thread before their stores.
template <typename Map>
__device__ __forceinline__ void stage_f4(const float4* __restrict__ src, int n, int valid, Map map) {
  for (int base = threadIdx.x; base < n; base += 256 * 8) {
    float4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int e = base + 256 * t;
      v[t] = e < valid ? src[e] : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int e = base + 256 * t;
      if (e < n) *map(e) = v[t];
    }
  }
}

__global__ __launch_bounds__(256) void gate_scores_kernel(const ScoreParams p) {
  extern __shared__ float lds[];
  const int bg = blockIdx.z;
  const int i0 = blockIdx.x * kTI, j0 = blockIdx.y * kTJ;
  const int tid = threadIdx.x;
  const int jl = tid & 63, ig = tid >> 6;
  const int krow = p.Pk * p.P + 4;  // padded key row (floats), keeps lanes on distinct banks
  const int j = j0 + jl;
  float* out = p.scores + (int64_t)bg * p.Qb * p.Kb;
  if (p.causal && j0 > i0 + kTI - 1) {
    // Entirely above the diagonal.
    for (int r = 0; r < kRowsPerWave; ++r) {
      const int i = i0 + ig * kRowsPerWave + r;
      if (i < p.Qb && j < p.Kb) out[(int64_t)i * p.Kb + j] = -INFINITY;
    }
    return;
  }
  float* qs = lds;                          // [kTI][Pq*P]
  float* ks = lds + kTI * p.Pq * p.P;       // [kTJ][krow]
  const int qrow = p.Pq * p.P;
  {
    const int rows = p.Qb - i0 < kTI ? p.Qb - i0 : kTI;
    const float4* src = reinterpret_cast<const float4*>(p.qp + ((int64_t)bg * p.Qb + i0) * qrow);
    float4* dst = reinterpret_cast<float4*>(qs);
    stage_f4(src, kTI * qrow / 4, rows * qrow / 4, [&](int e) { return dst + e; });
  }
  const int kr = p.Pk * p.P, kr4 = kr / 4;
  {
    const int rows = p.Kb - j0 < kTJ ? p.Kb - j0 : kTJ;
    const float4* src = reinterpret_cast<const float4*>(p.kp + ((int64_t)bg * p.Kb + j0) * kr);
    stage_f4(src, kTJ * kr4, rows * kr4, [&](int e) {
      const int r = e / kr4;
      return reinterpret_cast<float4*>(ks + r * krow + 4 * (e - r * kr4));
    });
  }
  __syncthreads();
  const float* qw = qs + ig * kRowsPerWave * qrow;
  float best[kRowsPerWave];
  for (int a = 0; a < p.Pq; ++a)
    for (int c = 0; c < p.Pk; ++c) {
      float acc[kRowsPerWave];
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) acc[r] = 0.f;
      const float* kv = ks + jl * krow + c * p.P;
#pragma unroll 8
      for (int e = 0; e < p.P; e += 4) {
        const float4 y = *reinterpret_cast<const float4*>(kv + e);
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
          const float4 x = *reinterpret_cast<const float4*>(qw + r * qrow + a * p.P + e);
          acc[r] = __builtin_fmaf(x.x, y.x, acc[r]);
          acc[r] = __builtin_fmaf(x.y, y.y, acc[r]);
          acc[r] = __builtin_fmaf(x.z, y.z, acc[r]);
          acc[r] = __builtin_fmaf(x.w, y.w, acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r)
        best[r] = (a == 0 && c == 0) ? acc[r] : (acc[r] > best[r] ? acc[r] : best[r]);
    }
  for (int r = 0; r < kRowsPerWave; ++r) {
    const int i = i0 + ig * kRowsPerWave + r;
    if (i < p.Qb && j < p.Kb) out[(int64_t)i * p.Kb + j] = (!p.causal || j <= i) ? best[r] / p.div : -INFINITY;
  }
}

// The same scores, register-blocked, for one query prototype and PK (1 or 2)
// key prototypes: a workgroup covers 16TR query blocks x 64 key blocks and
// thread (tr, tc) holds query blocks TR*tr..TR*tr+TR-1 x key blocks
// 4tc..4tc+3 for every key prototype. The prototypes are staged transposed
// ([e][block]) in slices of kGS dims, so each step over e reads TR query
// values and PK float4 of key values for 4 * TR * PK fmaf (the kernel above
// reads five float4 for 16). Same operation order as the kernel above.
constexpr int kGT = 64, kGS = 32;  // key tile, slice of the projection dim
constexpr int kScoreTR = 2;        // query blocks per thread (tile of 16 * kScoreTR)
template <int PK, int TR>
__global__ __launch_bounds__(256) void gate_scores_tile_kernel(const ScoreParams p) {
  constexpr int R = 16 * TR;               // query blocks per tile
  constexpr int kXRow = R + 4, kYRow = kGT + 4;  // padded LDS rows (floats)
  constexpr int kBands = kGT / R;          // query tiles per 64-block band
  __shared__ __attribute__((aligned(16))) float xs[kGS * kXRow];
  __shared__ __attribute__((aligned(16))) float ys[PK * kGS * kYRow];
  int bg, i0, j0;
  if (p.causal == 2) {
    // 1-D grid over the tiles on or below the diagonal (Qb == Kb).  Band m
    // (query blocks 64m..64m+63) holds kBands query tiles of m + 1 key tiles
    // each, kBands * m(m+1)/2 tiles before it.
    const int nt = (p.Qb + kGT - 1) / kGT, ntri = kBands * (nt * (nt + 1) / 2);
    bg = blockIdx.x / ntri;
    const int t = blockIdx.x - bg * ntri;
    int m = (int)((sqrtf(8.f * (float)t / kBands + 1.f) - 1.f) * 0.5f);
    while (kBands * ((m + 1) * (m + 2) / 2) <= t) ++m;
    while (kBands * (m * (m + 1) / 2) > t) --m;
    const int rem = t - kBands * (m * (m + 1) / 2);
    const int h = rem / (m + 1);
    i0 = (m * kBands + h) * R;
    j0 = (rem - h * (m + 1)) * kGT;
  } else {
    bg = blockIdx.z;
    i0 = blockIdx.x * R;
    j0 = blockIdx.y * kGT;
  }
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  float* out = p.scores + (int64_t)bg * p.Qb * p.Kb;
  if (p.causal && j0 > i0 + R - 1) {
    // Entirely above the diagonal.
    for (int r = 0; r < TR; ++r) {
      const int i = i0 + TR * tr + r;
      for (int k = 0; k < 4; ++k) {
        const int j = j0 + 4 * tc + k;
        if (i < p.Qb && j < p.Kb) out[(int64_t)i * p.Kb + j] = -INFINITY;
      }
    }
    return;
  }
  const float* qsrc = p.qp + (int64_t)bg * p.Qb * p.P;
  const float* ksrc = p.kp + (int64_t)bg * p.Kb * PK * p.P;
  float acc[PK][TR][4];
#pragma unroll
  for (int c = 0; c < PK; ++c)
#pragma unroll
    for (int r = 0; r < TR; ++r)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[c][r][k] = 0.f;
  // Staging map: kD4 consecutive lanes read one block's slice (contiguous).
  constexpr int kD4 = kGS / 4;                  // float4 per block slice
  constexpr int kLoadsQ = R * kD4 / 256;        // query float4 per thread
  constexpr int kLoads = kGT * kD4 / 256;       // key float4 per thread per prototype
  // The next slice's operands are loaded into registers while the current
  // slice is consumed from LDS.
  float4 qv[kLoadsQ], kv[PK][kLoads];
  auto load_slice = [&](int e0) {
#pragma unroll
    for (int t = 0; t < kLoadsQ; ++t) {
      const int idx = tid + 256 * t, blk = idx / kD4, d4 = idx % kD4;
      const int i = i0 + blk;
      qv[t] = i < p.Qb ? *reinterpret_cast<const float4*>(qsrc + (int64_t)i * p.P + e0 + 4 * d4)
                       : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int t = 0; t < kLoads; ++t) {
      const int idx = tid + 256 * t, blk = idx / kD4, d4 = idx % kD4;
      const int j = j0 + blk;
#pragma unroll
      for (int c = 0; c < PK; ++c)
        kv[c][t] = j < p.Kb ? *reinterpret_cast<const float4*>(ksrc + ((int64_t)j * PK + c) * p.P + e0 + 4 * d4)
                            : float4{0.f, 0.f, 0.f, 0.f};
    }
  };
  load_slice(0);
  for (int e0 = 0; e0 < p.P; e0 += kGS) {
    __syncthreads();  // the previous slice has been read
#pragma unroll
    for (int t = 0; t < kLoadsQ; ++t) {
      const int idx = tid + 256 * t, blk = idx / kD4, d4 = idx % kD4;
      float* x = xs + 4 * d4 * kXRow + blk;
      x[0] = qv[t].x;
      x[kXRow] = qv[t].y;
      x[2 * kXRow] = qv[t].z;
      x[3 * kXRow] = qv[t].w;
    }
#pragma unroll
    for (int t = 0; t < kLoads; ++t) {
      const int idx = tid + 256 * t, blk = idx / kD4, d4 = idx % kD4;
#pragma unroll
      for (int c = 0; c < PK; ++c) {
        float* y = ys + (c * kGS + 4 * d4) * kYRow + blk;
        y[0] = kv[c][t].x;
        y[kYRow] = kv[c][t].y;
        y[2 * kYRow] = kv[c][t].z;
        y[3 * kYRow] = kv[c][t].w;
      }
    }
    __syncthreads();
    if (e0 + kGS < p.P) load_slice(e0 + kGS);
#pragma unroll 8
    for (int e = 0; e < kGS; ++e) {
      float x[TR];
#pragma unroll
      for (int r = 0; r < TR; r += 2) {
        const float2 x2 = *reinterpret_cast<const float2*>(xs + e * kXRow + TR * tr + r);
        x[r] = x2.x;
        x[r + 1] = x2.y;
      }
#pragma unroll
      for (int c = 0; c < PK; ++c) {
        const float4 y4 = *reinterpret_cast<const float4*>(ys + (c * kGS + e) * kYRow + 4 * tc);
        const float y[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
          for (int k = 0; k < 4; ++k) acc[c][r][k] = __builtin_fmaf(x[r], y[k], acc[c][r][k]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < TR; ++r) {
    const int i = i0 + TR * tr + r;
    if (i >= p.Qb) continue;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = j0 + 4 * tc + k;
      float best = acc[0][r][k];
#pragma unroll
      for (int c = 1; c < PK; ++c) best = acc[c][r][k] > best ? acc[c][r][k] : best;
      v[k] = (!p.causal || j <= i) ? best / p.div : -INFINITY;
    }
    float* o = out + (int64_t)i * p.Kb + j0 + 4 * tc;
    if (j0 + 4 * tc + 3 < p.Kb && (p.Kb & 3) == 0) {
      *reinterpret_cast<float4*>(o) = float4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (j0 + 4 * tc + k < p.Kb) o[k] = v[k];
    }
  }
}

// The same scores for prototype counts whose tiles do not fit in LDS (e.g.
// 8 x 8 prototypes of 128 dims): one thread per score, operands read through
// the cache, identical operation order.
__global__ __launch_bounds__(256) void gate_scores_direct_kernel(const ScoreParams p, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int j = (int)(idx % p.Kb);
  const int64_t r = idx / p.Kb;
  const int i = (int)(r % p.Qb);
  const int64_t bg = r / p.Qb;
  float v = -INFINITY;
  if (!p.causal || j <= i) {
    const float* qrow = p.qp + (bg * p.Qb + i) * (int64_t)p.Pq * p.P;
    const float* krow = p.kp + (bg * p.Kb + j) * (int64_t)p.Pk * p.P;
    float best = 0.f;
    for (int a = 0; a < p.Pq; ++a)
      for (int c = 0; c < p.Pk; ++c) {
        const float4* x = reinterpret_cast<const float4*>(qrow + a * p.P);
        const float4* y = reinterpret_cast<const float4*>(krow + c * p.P);
        float acc = 0.f;
#pragma unroll 4
        for (int e = 0; e < p.P / 4; ++e) {
          const float4 xv = x[e], yv = y[e];
          acc = __builtin_fmaf(xv.x, yv.x, acc);
          acc = __builtin_fmaf(xv.y, yv.y, acc);
          acc = __builtin_fmaf(xv.z, yv.z, acc);
          acc = __builtin_fmaf(xv.w, yv.w, acc);
        }
        best = (a == 0 && c == 0) ? acc : (acc > best ? acc : best);
      }
    v = best / p.div;
  }
  p.scores[idx] = v;
}

// Causal top-k per row: radix select (4 passes of 8 bits over order keys) for
// the k-th largest key, then an in-order compaction that takes every larger key
// and the lowest-index entries equal to it.  One workgroup per row.
constexpr int kTopkMaxKb = 8192;
__global__ __launch_bounds__(256) void causal_topk_kernel(const float* __restrict__ scores, int Qb, int Kb, int k,
                                                          int32_t* __restrict__ out) {
  __shared__ uint32_t keys[kTopkMaxKb];
  __shared__ int hist[256];
  __shared__ int sel_bin, sel_rem;
  const int row = blockIdx.x;  // r * Qb + i
  const int i = row % Qb;
  const int tid = threadIdx.x;
  const int n = i + 1 < Kb ? i + 1 : Kb;
  int32_t* o = out + (int64_t)row * k;
  if (n <= k) {
    for (int t = tid; t < k; t += 256) o[t] = t < n ? t : -1;
    return;
  }
  const float* srow = scores + (int64_t)row * Kb;
  for (int j = tid; j < n; j += 256) keys[j] = order_key(srow[j] + 0.0f);  // -0 -> +0
  uint32_t prefix = 0, mask = 0;
  int rem = k;
  for (int pass = 3; pass >= 0; --pass) {
    hist[tid] = 0;
    __syncthreads();
    const int sh = 8 * pass;
    for (int j = tid; j < n; j += 256)
      if ((keys[j] & mask) == prefix) atomicAdd(&hist[(keys[j] >> sh) & 255], 1);
    __syncthreads();
    if (tid < 64) {
      // The bin holding the rem-th largest key, counting from bin 255 down:
      // lane l takes bins 255 - 4l .. 252 - 4l, the lanes' counts are
      // prefix-summed from the top, and the lane whose range holds rank rem
      // finds the bin (the same bin and remainder as a scan from the top).
      const int b0 = 255 - 4 * tid;
      const int c0 = hist[b0], c1 = hist[b0 - 1], c2 = hist[b0 - 2], c3 = hist[b0 - 3];
      const int own = c0 + c1 + c2 + c3;
      int incl = own;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off);
        if (tid >= off) incl += t;
      }
      int cum = incl - own;  // keys in the bins above this lane's
      if (cum < rem && rem <= incl) {
        int bin = b0;
        if (cum + c0 < rem) {
          cum += c0;
          bin = b0 - 1;
          if (cum + c1 < rem) {
            cum += c1;
            bin = b0 - 2;
            if (cum + c2 < rem) {
              cum += c2;
              bin = b0 - 3;
            }
          }
        }
        sel_bin = bin;
        sel_rem = rem - cum;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sel_bin << sh;
    mask |= 255u << sh;
    rem = sel_rem;
    __syncthreads();
  }
  // prefix = key of the k-th largest; take `rem` of the entries equal to it.
  if (tid < 64) {
    const uint32_t thr = prefix;
    int eq_base = 0, out_base = 0;
    const uint64_t lt = (tid == 0) ? 0ull : (~0ull >> (64 - tid));
    for (int c0 = 0; c0 < n; c0 += 64) {
      const int j = c0 + tid;
      const uint32_t key = j < n ? keys[j] : 0u;
      const bool eq = j < n && key == thr;
      const uint64_t eqb = __ballot(eq);
      const int rank = eq_base + __popcll(eqb & lt);
      const bool sel = j < n && (key > thr || (eq && rank < rem));
      const uint64_t sb = __ballot(sel);
      if (sel) o[out_base + __popcll(sb & lt)] = j;
      eq_base += __popcll(eqb);
      out_base += __popcll(sb);
    }
  }
}

// Causal top-k with one wavefront per row (rows up to kWaveTopkKb keys): each
// lane holds keys j = lane + 64 s in registers.  A 32-step binary search over
// order keys finds the k-th largest key T (the largest T with at least k keys
// >= T), counting with ballots, or any T with exactly k keys >= T; then an
// in-order compaction takes every key above T and the lowest-index keys equal
// to it.  Same result as causal_topk_kernel, without LDS atomics or
// workgroup barriers.
constexpr int kWaveTopkKb = 1024;
constexpr int kWaveTopkPer = kWaveTopkKb / 64;
//
// One wavefront selects the top k of srow[0..n) (n <= kWaveTopkKb) into o;
// cw is 64 words of LDS private to the wavefront.  srow may be global or LDS.
__device__ __forceinline__ void topk_row_wave(const float* __restrict__ srow, int n, int k, int32_t* __restrict__ o,
                                              uint32_t* cw) {
  const int lane = threadIdx.x & 63;
  if (n <= k) {
    for (int t = lane; t < k; t += 64) o[t] = t < n ? t : -1;
    return;
  }
  uint32_t key[kWaveTopkPer];
#pragma unroll
  for (int s = 0; s < kWaveTopkPer; ++s) {
    const int j = lane + 64 * s;
    key[s] = j < n ? order_key(srow[j] + 0.0f) : 0u;  // -0 -> +0; absent keys rank below all
  }
  // The search stops early once exactly k keys are >= the candidate: those k
  // keys are then the top k (the k-th largest is >= it and the (k+1)-th is
  // below), and the compaction below takes exactly them, as it would with the
  // k-th largest key itself as T.
  //
  // First a cheap bound: t0 = the k-th largest of the 64 lane maxima (k <=
  // 64), so at least k keys are >= t0 and the k-th largest key T is >= t0.
  // When at most 64 keys are >= t0 they are compacted into one slot per lane
  // and T is searched among them: for every candidate value >= t0 their count
  // equals the count over all keys, and below t0 both are >= k, so the search
  // ends at the same T (the early exit is taken only at or above t0).
  // Otherwise the search runs over all 16 slots.
  uint32_t T = 0;
  int nc = kWaveTopkKb + 1;
  uint32_t t0 = 0;
  if (k <= 64) {
    uint32_t lmax = key[0];
#pragma unroll
    for (int s = 1; s < kWaveTopkPer; ++s) lmax = key[s] > lmax ? key[s] : lmax;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = t0 | (1u << bit);
      if (__popcll(__ballot(lmax >= cand)) >= k) t0 = cand;
    }
    nc = 0;
#pragma unroll
    for (int s = 0; s < kWaveTopkPer; ++s) nc += __popcll(__ballot(key[s] >= t0));
  }
  if (nc <= 64) {
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int base = 0;
#pragma unroll
    for (int s = 0; s < kWaveTopkPer; ++s) {
      const bool c = key[s] >= t0;
      const uint64_t b = __ballot(c);
      if (c) cw[base + __popcll(b & below)] = key[s];
      base += __popcll(b);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t ck = lane < nc ? cw[lane] : 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = T | (1u << bit);
      const int cnt = __popcll(__ballot(ck >= cand));
      if (cnt >= k) T = cand;
      if (cnt == k && cand >= t0) break;
    }
  } else {
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = T | (1u << bit);
      int cnt = 0;
#pragma unroll
      for (int s = 0; s < kWaveTopkPer; ++s) cnt += __popcll(__ballot(key[s] >= cand));
      if (cnt >= k) T = cand;
      if (cnt == k) break;
    }
  }
  int gt = 0;
#pragma unroll
  for (int s = 0; s < kWaveTopkPer; ++s) gt += __popcll(__ballot(key[s] > T));
  const int rem = k - gt;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int eq_base = 0, out_base = 0;
#pragma unroll
  for (int s = 0; s < kWaveTopkPer; ++s) {
    const int j = lane + 64 * s;
    const bool valid = j < n;
    const bool eq = valid && key[s] == T;
    const uint64_t eqb = __ballot(eq);
    const int rank = eq_base + __popcll(eqb & lt);
    const bool sel = valid && (key[s] > T || (eq && rank < rem));
    const uint64_t sb = __ballot(sel);
    if (sel) o[out_base + __popcll(sb & lt)] = j;
    eq_base += __popcll(eqb);
    out_base += __popcll(sb);
  }
}

__global__ __launch_bounds__(256) void causal_topk_wave_kernel(const float* __restrict__ scores, int64_t rows,
                                                               int Qb, int Kb, int k, int32_t* __restrict__ out) {
  __shared__ uint32_t cands[4][64];
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefront; no block barrier follows
  const int i = (int)(row % Qb);
  const int n = i + 1 < Kb ? i + 1 : Kb;
  topk_row_wave(scores + row * Kb, n, k, out + row * k, cands[threadIdx.x >> 6]);
}


// ---------------------------------------------------------------------------
// Fused flat selector for the deployed shape: head_dim 128, projection dim
// 128, 16-bit inputs, at most kPoolMaxG query heads per KV head and at most
// kWaveTopkKb key blocks.  Two launches instead of four, with every value
// produced by the operation sequences stated at the top of this file, so the
// selected blocks are identical to those of the four-kernel route.
//
// Block pooling here gives each wavefront a whole 64-token block: lane =
// 16 * lo + chunk (chunk = 8 dims, lo = 0..3), and the lane carries the four
// token lanes l = lo + 4m (m = 0..3) of block_pool_fast_kernel at D = 128
// (token t of a block in token lane t % 16, the 4 tokens of a token lane
// folded in order), so every wavefront load reads 4 consecutive tokens x 256
// contiguous bytes.  The halving tree over token lanes adds the same pairs:
// st = 8 and 4 inside a lane (m + 2, then m + 1), st = 2 and 1 across lanes
// (lane + 32, then lane + 16).
constexpr int kFD = 128;                   // head_dim of the fused route
constexpr int kFP = 128;                   // projection dim of the fused route
constexpr int kFLanes = 16, kFPer = 4;     // pool_lanes(kFD / 8) and 64 / kFLanes
constexpr int kFRows = 4;                  // query blocks per tile of the rows kernel
static_assert(pool_lanes(kFD / 8) == kFLanes && kSelBlock / kFLanes == kFPer, "fused pooling shape");

// Pins v in a register at this point: the sums of a token step are then
// computed when the step is consumed, not sunk to their use after the
// following steps' loads (which would keep every load's registers live).
// An empty asm statement: no instruction is emitted.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ...
// lds): lane l's bytes land at lds + 16 l.
__device__ __forceinline__ void sel_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Copies a [kFD][kFP] float32 weight matrix (64 KB) into LDS, 1 KB per
// wavefront instruction, shared among nwaves wavefronts (wave = 0..nwaves-1).
__device__ __forceinline__ void stage_weights(const float* w, float* lds, int wave, int nwaves) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(w), (short)0, kFD * kFP * 4, 0x00020000);
  const int lane = threadIdx.x & 63;
  for (int j = wave; j < kFD * kFP / 256; j += nwaves) sel_load_lds16(r, lds + 256 * j, 1024 * j + 16 * lane);
}

// Token of step (i, m) for lane group lo: token lane lo + 4m, i-th token of it.
__device__ __forceinline__ int fused_token(int lo, int m, int i) { return lo + 4 * m + kFLanes * i; }

// acc[m] holds token lane lo + 4m; leaves the block sum in lanes 0..15 (lo = 0).
__device__ __forceinline__ void fused_tree_sum(float (&acc)[4][8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[0][e] = acc[0][e] + acc[2][e];   // st = 8
    acc[1][e] = acc[1][e] + acc[3][e];
    acc[0][e] = acc[0][e] + acc[1][e];   // st = 4
    acc[0][e] = acc[0][e] + __shfl_down(acc[0][e], 32);  // st = 2
    acc[0][e] = acc[0][e] + __shfl_down(acc[0][e], 16);  // st = 1
  }
}

__device__ __forceinline__ void fused_tree_max(float (&mx)[4][8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    mx[0][e] = max_total(mx[0][e], mx[2][e]);
    mx[1][e] = max_total(mx[1][e], mx[3][e]);
    mx[0][e] = max_total(mx[0][e], mx[1][e]);
    mx[0][e] = max_total(mx[0][e], __shfl_down(mx[0][e], 32));
    mx[0][e] = max_total(mx[0][e], __shfl_down(mx[0][e], 16));
  }
}

struct SelKeysParams {
  const void* k;
  int64_t ks[4];
  const float* wk;  // [kFD][kFP]
  float* kp4;       // [BG][2][kFP / 4][nb][4]
  int Hkv, T, nb, tiles;  // tiles = ceil(nb / kKeyBlocks) per (batch, KV head)
};

constexpr int kKeyBlocks = 8;  // key blocks per workgroup of select_keys_kernel, 2 per wavefront

// Key side: one workgroup pools 8 key blocks of one (batch, KV head), two per
// wavefront -- block mean and per-dim max -- and projects the 16 pooled rows
// (fmaf chain over d from 0) with the weights staged in LDS, writing
// kp4[bg][c][e / 4][j][e % 4] (c = 0 mean, 1 max).
template <typename TIn>
__global__ __launch_bounds__(256) void select_keys_kernel(const SelKeysParams p) {
  __shared__ __attribute__((aligned(16))) float rows[2 * kKeyBlocks][kFD];  // row 2 * block + c
  __shared__ __attribute__((aligned(16))) float wl[kFD][kFP];               // the key projection
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = lane & 15, lo = lane >> 4;
  // (batch, KV head) fastest: the workgroups running together read all KV
  // heads of the same tokens (rows that are adjacent in [B, T, H, D] storage).
  const int BG = (int)(gridDim.x / p.tiles);
  const int bg = blockIdx.x % BG;
  const int j0 = (blockIdx.x / BG) * kKeyBlocks;
  const int b = bg / p.Hkv, g = bg - (bg / p.Hkv) * p.Hkv;
  const char* kb = static_cast<const char*>(p.k) +
                   ((int64_t)b * p.ks[0] + (int64_t)g * p.ks[1] + 8 * ch) * TIn::bytes;
  // All 32 loads of the wavefront's two blocks first (blocks and tokens
  // clamped into the tensor so no load is conditional; tokens past T are
  // replaced by zero when summed), then the weights into LDS.
  Raw8<TIn> kr[2][kFPer][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    int blk = j0 + 2 * wave + u;
    blk = blk < p.nb ? blk : p.nb - 1;
#pragma unroll
    for (int i = 0; i < kFPer; ++i)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int t = blk * kSelBlock + fused_token(lo, m, i);
        kr[u][i][m] = raw8_at<TIn>(kb, (int64_t)(t < p.T ? t : p.T - 1) * p.ks[2]);
      }
  }
  stage_weights(p.wk, &wl[0][0], wave, 4);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int blk = j0 + 2 * wave + u;
    if (blk >= p.nb) break;
    const int t0 = blk * kSelBlock;
    float acc[4][8], mx[4][8];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx[m][e] = -INFINITY;
#pragma unroll
    for (int i = 0; i < kFPer; ++i)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const bool valid = t0 + fused_token(lo, m, i) < p.T;
        float s[8];
        widen8<TIn>(kr[u][i][m], s);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          mx[m][e] = valid ? max_total(mx[m][e], s[e]) : mx[m][e];
          s[e] = valid ? s[e] : 0.f;
          acc[m][e] = (i == 0) ? s[e] : acc[m][e] + s[e];
        }
      }
    fused_tree_sum(acc);
    fused_tree_max(mx);
    if (lane < 16) {
      const int n = p.T - t0 < kSelBlock ? p.T - t0 : kSelBlock;
      const float den = (float)n;
      const int r = 2 * (2 * wave + u);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        rows[r][8 * ch + e] = acc[0][e] / den;
        rows[r + 1][8 * ch + e] = mx[0][e];
      }
    }
  }
  // Every wave's share of the weights is in LDS before the barrier.  The
  // barrier's release fence already waits for this wave's loads into LDS; the
  // explicit s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15) states it.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  // Projection: thread = output dim e, rows 8 * half .. 8 * half + 7.
  const int e = tid & (kFP - 1), half = tid >> 7;
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int d0 = 0; d0 < kFD; d0 += 4) {
    const float w0 = wl[d0][e], w1 = wl[d0 + 1][e], w2 = wl[d0 + 2][e], w3 = wl[d0 + 3][e];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float4 x = *reinterpret_cast<const float4*>(&rows[8 * half + r][d0]);
      a[r] = __builtin_fmaf(x.x, w0, a[r]);
      a[r] = __builtin_fmaf(x.y, w1, a[r]);
      a[r] = __builtin_fmaf(x.z, w2, a[r]);
      a[r] = __builtin_fmaf(x.w, w3, a[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int row = 8 * half + r, j = j0 + (row >> 1), c = row & 1;
    if (j < p.nb) p.kp4[((((int64_t)bg * 2 + c) * (kFP / 4) + (e >> 2)) * p.nb + j) * 4 + (e & 3)] = a[r];
  }
}

// ---------------------------------------------------------------------------
// Pooling and projection of the selector's query and key blocks in one
// persistent launch (head_dim = projection dim = 128, 16-bit inputs, G <= 8):
// the values of spruce_selector_pool followed by spruce_gate_project2, without
// the pooled summaries' round trip through HBM or the projection launch.
// Every wavefront takes (batch, KV head, block) tasks on its own (no
// workgroup barrier after the weights are staged): it pools the query block
// (G heads summed per token, block mean) and the key block (mean and per-dim
// max) with the token-lane order and trees of select_keys_kernel, then
// projects the three rows (fmaf chains over d from 0) with both weight
// matrices in LDS.  A two-slot ring holds the G query loads and the key load
// of a token step; consuming step s issues step s + 2, so 2(G + 1) loads per
// lane stay in flight, 8 wavefronts per CU.
struct PoolProjParams {
  const void* q;
  const void* k;
  int64_t qs[4], ks[4];
  const float* wq;  // [kFD][kFP]
  const float* wk;  // [kFD][kFP]
  float* qp;        // [BG][nb][kFP]
  float* kp;        // [BG][nb][2][kFP]
  int Hkv, T, nb, BG, ntasks;
  int qslice, kslice;  // bytes spanned by one (batch, KV group) slice of q / k
};

template <typename TIn, int G>
__global__ __launch_bounds__(512) void pool_project_kernel(const PoolProjParams p) {
  __shared__ __attribute__((aligned(16))) float wql[kFD][kFP];
  __shared__ __attribute__((aligned(16))) float wkl[kFD][kFP];
  __shared__ __attribute__((aligned(16))) float rowbuf[8][3][kFD];  // per wave: q mean, k mean, k max
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = lane & 15, lo = lane >> 4;
  stage_weights(p.wq, &wql[0][0], wave, 8);
  stage_weights(p.wk, &wkl[0][0], wave, 8);
  // The barrier's release fence waits for this wave's loads into LDS; the
  // explicit s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15) states it.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  const int nw = (int)gridDim.x * 8;
  const int w0 = (int)blockIdx.x * 8 + wave;
  const int mine = (p.ntasks - w0 + nw - 1) / nw;  // tasks w0, w0 + nw, ... (0 when w0 >= ntasks)
  if (mine <= 0) return;
  Raw8<TIn> qr[2][G], kr[2];
  float aq[4][8], ak[4][8], mk[4][8];
  auto task_of = [&](int n, int& bg, int& blk) __attribute__((always_inline)) {
    const int tau = w0 + n * nw;
    bg = tau % p.BG;  // (batch, KV head) fastest: the waves running together read neighbouring rows
    blk = tau / p.BG;
  };
  auto issue = [&](int n, int st) __attribute__((always_inline)) {
    n = n < mine ? n : mine - 1;  // past the last task: a repeated load, never consumed
    int bg, blk;
    task_of(n, bg, blk);
    const int i = st >> 2, m = st & 3;
    int t = blk * kSelBlock + fused_token(lo, m, i);
    t = t < p.T ? t : p.T - 1;
    const int b = bg / p.Hkv, g = bg - (bg / p.Hkv) * p.Hkv;
    const char* qb = static_cast<const char*>(p.q) + ((int64_t)b * p.qs[0] + (int64_t)(g * G) * p.qs[1]) * 2;
    const char* kb = static_cast<const char*>(p.k) + ((int64_t)b * p.ks[0] + (int64_t)g * p.ks[1]) * 2;
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(qb), (short)0, p.qslice, 0x00020000);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb), (short)0, p.kslice, 0x00020000);
    const int qoff = (int)(((int64_t)t * p.qs[2] + 8 * ch) * 2);
    const int koff = (int)(((int64_t)t * p.ks[2] + 8 * ch) * 2);
    const int sl = st & 1;
#pragma unroll
    for (int h = 0; h < G; ++h)
      qr[sl][h].a = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, (int)((int64_t)h * p.qs[1] * 2), 0));
    kr[sl].a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff, 0, 0));
  };
  auto consume = [&](int n, int st) __attribute__((always_inline)) {
    int bg, blk;
    task_of(n, bg, blk);
    const int i = st >> 2, m = st & 3, sl = st & 1;
    const bool valid = blk * kSelBlock + fused_token(lo, m, i) < p.T;
    float s[8], x[8];
    widen8<TIn>(qr[sl][0], s);
#pragma unroll
    for (int h = 1; h < G; ++h) {
      widen8<TIn>(qr[sl][h], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = s[e] + x[e];
    }
    widen8<TIn>(kr[sl], x);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[e] = valid ? s[e] : 0.f;
      aq[m][e] = (i == 0) ? s[e] : aq[m][e] + s[e];
      const float mprev = (i == 0) ? -INFINITY : mk[m][e];
      mk[m][e] = valid ? max_total(mprev, x[e]) : mprev;
      x[e] = valid ? x[e] : 0.f;
      ak[m][e] = (i == 0) ? x[e] : ak[m][e] + x[e];
      pin(aq[m][e]);
      pin(ak[m][e]);
      pin(mk[m][e]);
    }
    __builtin_amdgcn_sched_barrier(0);  // slot sl is consumed before its next loads are issued
    if (st + 2 < 16) issue(n, st + 2);
    else issue(n + 1, st + 2 - 16);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto finish = [&](int n) __attribute__((always_inline)) {
    int bg, blk;
    task_of(n, bg, blk);
    fused_tree_sum(aq);
    fused_tree_sum(ak);
    fused_tree_max(mk);
    if (lane < 16) {
      const int t0 = blk * kSelBlock;
      const int cnt = p.T - t0 < kSelBlock ? p.T - t0 : kSelBlock;
      const float dq = (float)(G * cnt), dk = (float)cnt;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        rowbuf[wave][0][8 * ch + e] = aq[0][e] / dq;
        rowbuf[wave][1][8 * ch + e] = ak[0][e] / dk;
        rowbuf[wave][2][8 * ch + e] = mk[0][e];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float a[3][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
#pragma unroll 2
    for (int d0 = 0; d0 < kFD; d0 += 4) {
      float4 xr[3];
#pragma unroll
      for (int r = 0; r < 3; ++r) xr[r] = *reinterpret_cast<const float4*>(&rowbuf[wave][r][d0]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float wq0 = wql[d0 + u][lane], wq1 = wql[d0 + u][64 + lane];
        const float wk0 = wkl[d0 + u][lane], wk1 = wkl[d0 + u][64 + lane];
        const float xq = u == 0 ? xr[0].x : u == 1 ? xr[0].y : u == 2 ? xr[0].z : xr[0].w;
        const float xm = u == 0 ? xr[1].x : u == 1 ? xr[1].y : u == 2 ? xr[1].z : xr[1].w;
        const float xx = u == 0 ? xr[2].x : u == 1 ? xr[2].y : u == 2 ? xr[2].z : xr[2].w;
        a[0][0] = __builtin_fmaf(xq, wq0, a[0][0]);
        a[0][1] = __builtin_fmaf(xq, wq1, a[0][1]);
        a[1][0] = __builtin_fmaf(xm, wk0, a[1][0]);
        a[1][1] = __builtin_fmaf(xm, wk1, a[1][1]);
        a[2][0] = __builtin_fmaf(xx, wk0, a[2][0]);
        a[2][1] = __builtin_fmaf(xx, wk1, a[2][1]);
      }
    }
    float* oq = p.qp + ((int64_t)bg * p.nb + blk) * kFP;
    float* ok = p.kp + ((int64_t)bg * p.nb + blk) * 2 * kFP;
    oq[lane] = a[0][0];
    oq[64 + lane] = a[0][1];
    ok[lane] = a[1][0];
    ok[64 + lane] = a[1][1];
    ok[kFP + lane] = a[2][0];
    ok[kFP + 64 + lane] = a[2][1];
    // The row buffer is rewritten by the next task's tree only after every
    // lane has read it here.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  issue(0, 0);
  issue(0, 1);
  for (int n = 0; n < mine; ++n) {
#pragma unroll
    for (int st = 0; st < 16; ++st) consume(n, st);
    finish(n);
  }
}

struct SelRowsParams {
  const void* q;
  int64_t qs[4];
  const float* wq;   // [kFD][kFP]
  const float* kp4;  // select_keys_kernel's output
  int32_t* out;      // [BG][nb][k]
  int Hkv, T, nb, k, BG, row_tiles, ntiles;
  int slice_bytes;  // bytes spanned by one (batch, KV group) slice of q
  float div;
};

// Query side, persistent: workgroup w takes tiles w, w + grid, ... of kFRows
// query blocks of one (batch, KV head), heaviest (latest) tiles first.  Waves
// 0-3 pool the next tile's query blocks, one block each (G heads summed per
// token, block mean; the same token-lane order as select_keys_kernel), while
// waves 4-7 take the current tile through projection, MaxSim scores against
// every causal key block and the wave top-k, all in LDS.  Each tile step has
// two phases (scores | top-k) ending in a workgroup barrier; the pool waves
// project their blocks themselves at the end of pooling.
template <typename TIn, int G>
__global__ __launch_bounds__(512) void select_rows_kernel(const SelRowsParams p) {
  __shared__ __attribute__((aligned(16))) float qm[kFRows][kFD];      // pooled query block of each pool wave
  __shared__ __attribute__((aligned(16))) float qp[2][kFRows][kFP];   // projected query blocks, double buffer
  __shared__ __attribute__((aligned(16))) float sc[kFRows][kWaveTopkKb];
  __shared__ __attribute__((aligned(16))) float wql[kFD][kFP];  // the query projection, staged once
  __shared__ uint32_t cands[4][64];
  // The wave index is taken through readfirstlane so that the pool / score
  // split below is a scalar branch: each wave runs only its own side's
  // barriers.
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grid = (int)gridDim.x;
  const int mine = (p.ntiles - (int)blockIdx.x + grid - 1) / grid;  // tiles of this workgroup (>= 1)
  auto tile_at = [&](int kk, int& bg, int& i0) __attribute__((always_inline)) {
    const int tau = (int)blockIdx.x + kk * grid;
    bg = tau % p.BG;
    i0 = (p.row_tiles - 1 - tau / p.BG) * kFRows;
  };

  if (wave < 4) {
    // ---- pool waves: wave w pools and projects block w of each tile (16
    // steps (i, m) of G loads), token steps i = 0..2 | 3 in the two phases.  The
    // ring holds the G loads of steps (i, m = 0..3); consuming step (i, m)
    // issues step (i + 1, m), so up to 4G loads per lane stay in flight,
    // across the phase barriers too (barriers do not wait for outstanding
    // global loads).  Loads are issued without
    // per-lane conditions (block and token clamped into the tensor; values
    // past T are replaced by zero when consumed) so the compiler waits for
    // each step's loads in issue order.
    const int ch = lane & 15, lo = lane >> 4;
    Raw8<TIn> ring[4][G];
    float acc[4][8];
    // Buffer loads from the (batch, KV group) slice: one 32-bit offset per
    // lane and step, the head offset in an SGPR (the host checks that a slice
    // spans less than 2^31 bytes).
    auto issue = [&](int tk, int i, int m) __attribute__((always_inline)) {
      tk = tk < mine ? tk : mine - 1;  // past the last tile: a repeated load, never consumed
      int bg, i0;
      tile_at(tk, bg, i0);
      int blk = i0 + wave;
      blk = blk < p.nb ? blk : p.nb - 1;
      int t = blk * kSelBlock + fused_token(lo, m, i);
      t = t < p.T ? t : p.T - 1;
      const int b = bg / p.Hkv, g = bg - (bg / p.Hkv) * p.Hkv;
      const char* base = static_cast<const char*>(p.q) + ((int64_t)b * p.qs[0] + (int64_t)(g * G) * p.qs[1]) * 2;
      const __amdgpu_buffer_rsrc_t r =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, p.slice_bytes, 0x00020000);
      const int voff = (int)(((int64_t)t * p.qs[2] + 8 * ch) * 2);
#pragma unroll
      for (int h = 0; h < G; ++h)
        ring[m][h].a = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, (int)((int64_t)h * p.qs[1] * 2), 0));
    };
    auto consume = [&](int tk, int i) __attribute__((always_inline)) {
      int bg, i0;
      tile_at(tk, bg, i0);
      const int blk = i0 + wave;
      const bool live = blk < p.nb;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        float s[8];
        widen8<TIn>(ring[m][0], s);
#pragma unroll
        for (int h = 1; h < G; ++h) {
          float x[8];
          widen8<TIn>(ring[m][h], x);
#pragma unroll
          for (int e = 0; e < 8; ++e) s[e] = s[e] + x[e];
        }
        const bool valid = live && blk * kSelBlock + fused_token(lo, m, i) < p.T;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s[e] = valid ? s[e] : 0.f;
          acc[m][e] = (i == 0) ? s[e] : acc[m][e] + s[e];
          pin(acc[m][e]);
        }
        // Slot m is consumed before its next loads are issued: the scheduler
        // may not hoist them (that would hold two rings of registers).
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < kFPer) issue(tk, i + 1, m);
        else issue(tk + 1, 0, m);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // The block mean goes through this wave's LDS row, then the wave projects
    // it (outputs lane and lane + 64, fmaf chain over d from 0) into qp[buf].
    auto finish = [&](int tk, int buf) __attribute__((always_inline)) {
      int bg, i0;
      tile_at(tk, bg, i0);
      const int blk = i0 + wave;
      if (blk >= p.nb) return;
      fused_tree_sum(acc);
      if (lane < 16) {
        const int t0 = blk * kSelBlock;
        const int n = p.T - t0 < kSelBlock ? p.T - t0 : kSelBlock;
        const float den = (float)(G * n);
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = acc[0][e] / den;
        float4* dst = reinterpret_cast<float4*>(&qm[wave][8 * ch]);
        dst[0] = float4{o[0], o[1], o[2], o[3]};
        dst[1] = float4{o[4], o[5], o[6], o[7]};
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float a0 = 0.f, a1 = 0.f;
#pragma unroll 4
      for (int d0 = 0; d0 < kFD; d0 += 4) {
        const float4 x = *reinterpret_cast<const float4*>(&qm[wave][d0]);
        a0 = __builtin_fmaf(x.x, wql[d0][lane], a0);
        a1 = __builtin_fmaf(x.x, wql[d0][64 + lane], a1);
        a0 = __builtin_fmaf(x.y, wql[d0 + 1][lane], a0);
        a1 = __builtin_fmaf(x.y, wql[d0 + 1][64 + lane], a1);
        a0 = __builtin_fmaf(x.z, wql[d0 + 2][lane], a0);
        a1 = __builtin_fmaf(x.z, wql[d0 + 2][64 + lane], a1);
        a0 = __builtin_fmaf(x.w, wql[d0 + 3][lane], a0);
        a1 = __builtin_fmaf(x.w, wql[d0 + 3][64 + lane], a1);
      }
      qp[buf][wave][lane] = a0;
      qp[buf][wave][64 + lane] = a1;
    };
    // Tile steps -1 .. mine - 2 pool tile step + 1; the last step pools
    // nothing.  Each tile's first token step is issued at the top of its
    // iteration, so no load is in flight across the loop's back edge (loads
    // carried there were copied between register sets after a full wait).
#pragma unroll
    for (int m = 0; m < 4; ++m) issue(0, 0, m);
    for (int nxt = 0; nxt < mine; ++nxt) {
      consume(nxt, 0);
      consume(nxt, 1);
      consume(nxt, 2);
      __syncthreads();
      consume(nxt, 3);
      finish(nxt, nxt & 1);
      __syncthreads();
    }
    __syncthreads();
    __syncthreads();
    return;
  }

  // ---- score waves
  const int sw = wave - 4;
  // The query projection into LDS, complete before the first barrier: the
  // pool waves read it after that barrier.  The barrier's release fence
  // already waits for this wave's loads into LDS; the explicit s_waitcnt
  // vmcnt(0) expcnt(7) lgkmcnt(15) states it.
  stage_weights(p.wq, &wql[0][0], sw, 4);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  for (int kk = -1; kk < mine; ++kk) {
    if (kk < 0) {
      __syncthreads();
      __syncthreads();
      continue;
    }
    int bg, i0;
    tile_at(kk, bg, i0);
    const int buf = kk & 1;
    // Phase 1: wave sw scores key blocks 256 sw .. 256 sw + 255 (4 per lane)
    // against the tile's query blocks; keys past the last row's diagonal are
    // not needed.
    const int nk = i0 + kFRows < p.nb ? i0 + kFRows : p.nb;
    const int jb = 256 * sw + 4 * lane;
    if (256 * sw < nk) {
      const float4* kp = reinterpret_cast<const float4*>(p.kp4) + (int64_t)bg * 2 * (kFP / 4) * p.nb;
      float acc[kFRows][4][2];
#pragma unroll
      for (int r = 0; r < kFRows; ++r)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[r][u][0] = acc[r][u][1] = 0.f;
      auto load_y = [&](int e4, float4 (&dst)[2][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            dst[c][u] = kp[((int64_t)c * (kFP / 4) + e4) * p.nb + (jb + u < p.nb ? jb + u : p.nb - 1)];
      };
      auto step = [&](int e4, const float4 (&y)[2][4]) __attribute__((always_inline)) {
        float4 x[kFRows];
#pragma unroll
        for (int r = 0; r < kFRows; ++r) x[r] = *reinterpret_cast<const float4*>(&qp[buf][r][4 * e4]);
#pragma unroll
        for (int r = 0; r < kFRows; ++r)
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              float a = acc[r][u][c];
              a = __builtin_fmaf(x[r].x, y[c][u].x, a);
              a = __builtin_fmaf(x[r].y, y[c][u].y, a);
              a = __builtin_fmaf(x[r].z, y[c][u].z, a);
              a = __builtin_fmaf(x[r].w, y[c][u].w, a);
              acc[r][u][c] = a;
            }
      };
      // Ring of four register sets: the keys of dims 4(e4 + 4) load while
      // those of dims 4 e4 are used (past the end a repeated load, unused).
      float4 yb[4][2][4];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) load_y(r4, yb[r4]);
      for (int e4 = 0; e4 < kFP / 4; e4 += 4) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          step(e4 + r4, yb[r4]);
          __builtin_amdgcn_sched_barrier(0);  // keep each set's reload right after its use
          load_y(e4 + r4 + 4 < kFP / 4 ? e4 + r4 + 4 : kFP / 4 - 1, yb[r4]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int r = 0; r < kFRows; ++r) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float best = acc[r][u][0];
          best = acc[r][u][1] > best ? acc[r][u][1] : best;
          v[u] = best / p.div;
        }
        if (jb < nk) *reinterpret_cast<float4*>(&sc[r][jb]) = float4{v[0], v[1], v[2], v[3]};
      }
    }
    __syncthreads();
    // Phase 2: wave sw selects the top k of query block i0 + sw.
    if (i0 + sw < p.nb) {
      const int i = i0 + sw;
      topk_row_wave(sc[sw], i + 1, p.k, p.out + ((int64_t)bg * p.nb + i) * p.k, cands[sw]);
    }
    __syncthreads();
  }
}

}  // namespace spruce

using namespace spruce;

extern "C" int spruce_selector_pool(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                    int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype,
                                    float* q_mean, float* k_sum, void* stream) {
  SPRUCE_REQUIRE(q || k, "nothing to pool: q and k are both NULL");
  SPRUCE_REQUIRE(B >= 1 && T >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "invalid shape");
  SPRUCE_REQUIRE(D >= 8 && D <= 2048 && D % 8 == 0, "head_dim must be a multiple of 8 (<= 2048), got %lld",
                 (long long)D);
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  SPRUCE_REQUIRE(!q || (qs && qs[3] == 1 && q_mean), "q needs strides with a contiguous last dim and q_mean");
  SPRUCE_REQUIRE(!k || (ks && ks[3] == 1 && k_sum), "k needs strides with a contiguous last dim and k_sum");
  const int per16 = dtype == SPRUCE_DTYPE_F32 ? 4 : 8;
  if (q) SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && qs[0] % per16 == 0 && qs[1] % per16 == 0 &&
                            qs[2] % per16 == 0, "q rows must be 16-byte aligned");
  if (k) SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(k) % 16 == 0 && ks[0] % per16 == 0 && ks[1] % per16 == 0 &&
                            ks[2] % per16 == 0, "k rows must be 16-byte aligned");
  PoolParams p{};
  p.q = q;
  p.k = k;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = q ? qs[i] : 0;
    p.ks[i] = k ? ks[i] : 0;
  }
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.T = (int)T;
  p.D = (int)D;
  p.G = (int)(Hq / Hkv);
  p.nb = (int)((T + kSelBlock - 1) / kSelBlock);
  p.dtype = dtype;
  p.q_mean = q_mean;
  p.k_sum = k_sum;
  const int64_t grid = B * Hkv * p.nb;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "grid too large");
  const int dch = (int)(D / 8);
  const int L = pool_lanes(dch);
  if (p.G <= kPoolMaxG && kSelBlock / L <= kPoolMaxPer) {
    if (dtype == SPRUCE_DTYPE_BF16)
      hipLaunchKernelGGL(block_pool_fast_kernel<InBF16>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, p);
    else if (dtype == SPRUCE_DTYPE_F16)
      hipLaunchKernelGGL(block_pool_fast_kernel<InF16>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, p);
    else
      hipLaunchKernelGGL(block_pool_fast_kernel<InF32>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, p);
    return check_launch("block_pool_fast_kernel");
  }
  hipLaunchKernelGGL(block_pool_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, p);
  return check_launch("block_pool_kernel");
}

extern "C" int spruce_gate_project(const float* x, const float* w, int64_t N, int64_t D, int64_t P, float* out,
                                   void* stream) {
  SPRUCE_REQUIRE(x && w && out, "x, w and out must be non-null");
  SPRUCE_REQUIRE(N >= 1 && D >= 1 && P >= 1 && N * P < ((int64_t)1 << 40), "invalid projection shape");
  const bool vec = D % 4 == 0 && P % 4 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0 &&
                   ((uintptr_t)out % 16) == 0;
  if (vec && N >= kBlockProjectRows) {
    constexpr int TR = kBlockProjectTR, TC = kBlockProjectTC;
    const int64_t brows = (N + 16 * TR - 1) / (16 * TR);
    SPRUCE_REQUIRE(brows < ((int64_t)1 << 31) && P < ((int64_t)1 << 20) && D < ((int64_t)1 << 20),
                   "projection too large");
    hipLaunchKernelGGL((project_block_kernel<TR, TC, ProjRowsF32>),
                       dim3((unsigned)brows, (unsigned)((P + 16 * TC - 1) / (16 * TC))), dim3(256), 0,
                       (hipStream_t)stream, ProjRowsF32{x}, w, N, (int)D, (int)P, out);
    return check_launch("project_block_kernel");
  }
  if (vec) {
    const int64_t vrows = (N + 63) / 64;
    SPRUCE_REQUIRE(vrows < ((int64_t)1 << 31) && P < ((int64_t)1 << 20) && D < ((int64_t)1 << 20),
                   "projection too large");
    const ProjPair pp{x, w, out, nullptr, nullptr, nullptr, N, 0, vrows, (int)D, (int)P};
    hipLaunchKernelGGL(project_tile_kernel<4>, dim3((unsigned)vrows, (unsigned)((P + kVC - 1) / kVC)), dim3(256), 0,
                       (hipStream_t)stream, pp);
    return check_launch("project_tile_kernel");
  }
  const int64_t rows = (N + kPR - 1) / kPR;
  SPRUCE_REQUIRE(rows < ((int64_t)1 << 31) && P < ((int64_t)1 << 20) && D < ((int64_t)1 << 20),
                 "projection too large");
  hipLaunchKernelGGL(project_kernel, dim3((unsigned)rows, (unsigned)((P + kPC - 1) / kPC)), dim3(256), 0,
                     (hipStream_t)stream, x, w, N, (int)D, (int)P, out);
  return check_launch("project_kernel");
}

extern "C" int spruce_gate_project_levels(const void* const* levels, const int64_t* level_nodes, int64_t nlevels,
                                          int64_t S, int64_t Pk, int64_t D, int dtype, const float* w, int64_t P,
                                          float* out, int layout, void* stream) {
  SPRUCE_REQUIRE(levels && level_nodes && w && out, "levels, level_nodes, w and out must be non-null");
  SPRUCE_REQUIRE(layout == SPRUCE_KP_ROWS || layout == SPRUCE_KP_INTERLEAVED, "unknown output layout %d", layout);
  SPRUCE_REQUIRE(nlevels >= 1 && nlevels <= kProjMaxSeg, "between 1 and %d levels, got %lld", kProjMaxSeg,
                 (long long)nlevels);
  SPRUCE_REQUIRE(S >= 1 && S < (1 << 20) && Pk >= 1 && Pk <= 1024 && D >= 4 && D <= 4096 && P >= 4 && P <= 4096,
                 "invalid projection shape");
  SPRUCE_REQUIRE(D % 4 == 0 && P % 4 == 0, "head_dim and projection dim must be multiples of 4");
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  const int eb = dtype == SPRUCE_DTYPE_F32 ? 4 : 2;
  SPRUCE_REQUIRE(((uintptr_t)w % 16) == 0 && ((uintptr_t)out % 16) == 0, "w and out must be 16-byte aligned");
  ProjSegs g{};
  g.nseg = (int)nlevels;
  g.P = (int)Pk;
  int64_t total = 0;
  for (int v = 0; v < nlevels; ++v) {
    SPRUCE_REQUIRE(levels[v] != nullptr && level_nodes[v] >= 1 && level_nodes[v] < ((int64_t)1 << 30),
                   "level %d: null buffer or node count out of range", v);
    SPRUCE_REQUIRE(((uintptr_t)levels[v] % (size_t)(4 * eb)) == 0, "level %d is not %d-byte aligned", v, 4 * eb);
    g.base[v] = levels[v];
    g.off[v] = total;
    total += level_nodes[v];
  }
  g.off[nlevels] = total;
  g.N = total;
  const int64_t N = S * total * Pk;
  SPRUCE_REQUIRE(N * P < ((int64_t)1 << 40), "projection too large");
  constexpr int TR = kBlockProjectTR, TC = kBlockProjectTC;
  const int64_t brows = (N + 16 * TR - 1) / (16 * TR);
  SPRUCE_REQUIRE(brows < ((int64_t)1 << 31), "projection too large");
  const dim3 grid((unsigned)brows, (unsigned)((P + 16 * TC - 1) / (16 * TC)));
  const hipStream_t st = (hipStream_t)stream;
  const bool il = layout == SPRUCE_KP_INTERLEAVED;
  auto go = [&](auto rows) {
    using RowsT = decltype(rows);
    if (il)
      hipLaunchKernelGGL((project_block_kernel<TR, TC, RowsT, true>), grid, dim3(256), 0, st, rows, w, N, (int)D,
                         (int)P, out, (int)Pk);
    else
      hipLaunchKernelGGL((project_block_kernel<TR, TC, RowsT, false>), grid, dim3(256), 0, st, rows, w, N, (int)D,
                         (int)P, out, 0);
  };
  if (dtype == SPRUCE_DTYPE_BF16)
    go(ProjRowsSeg<InBF16>{g});
  else if (dtype == SPRUCE_DTYPE_F16)
    go(ProjRowsSeg<InF16>{g});
  else
    go(ProjRowsSeg<InF32>{g});
  return check_launch("project_block_kernel");
}

// Both selector projections in one launch (32-row tiles: at the selector's
// sizes the single-problem launches leave most CUs idle); shapes outside the
// vector form or large enough for the block kernel take two launches.
extern "C" int spruce_gate_project2(const float* xa, const float* wa, int64_t Na, const float* xb, const float* wb,
                                    int64_t Nb, int64_t D, int64_t P, float* outa, float* outb, void* stream) {
  SPRUCE_REQUIRE(xa && wa && outa && xb && wb && outb, "x, w and out of both projections must be non-null");
  SPRUCE_REQUIRE(Na >= 1 && Nb >= 1 && D >= 1 && P >= 1 && (Na + Nb) * P < ((int64_t)1 << 40),
                 "invalid projection shape");
  auto aligned = [](const void* q) { return ((uintptr_t)q % 16) == 0; };
  const bool vec = D % 4 == 0 && P % 4 == 0 && aligned(xa) && aligned(wa) && aligned(outa) && aligned(xb) &&
                   aligned(wb) && aligned(outb);
  if (!vec || Na >= kBlockProjectRows || Nb >= kBlockProjectRows) {
    const int rc = spruce_gate_project(xa, wa, Na, D, P, outa, stream);
    return rc != 0 ? rc : spruce_gate_project(xb, wb, Nb, D, P, outb, stream);
  }
  SPRUCE_REQUIRE(P < ((int64_t)1 << 20) && D < ((int64_t)1 << 20), "projection too large");
  constexpr int TR = 2, R = 16 * TR;
  const int64_t ta = (Na + R - 1) / R, tb = (Nb + R - 1) / R;
  const ProjPair pp{xa, wa, outa, xb, wb, outb, Na, Nb, ta, (int)D, (int)P};
  hipLaunchKernelGGL(project_tile_kernel<TR>, dim3((unsigned)(ta + tb), (unsigned)((P + kVC - 1) / kVC)), dim3(256),
                     0, (hipStream_t)stream, pp);
  return check_launch("project_tile_kernel");
}

extern "C" int spruce_gate_scores(const float* qp, const float* kp, int64_t BG, int64_t Qb, int64_t Kb, int64_t Pq,
                                  int64_t Pk, int64_t P, float div, int causal, float* scores, void* stream) {
  SPRUCE_REQUIRE(qp && kp && scores, "qp, kp and scores must be non-null");
  SPRUCE_REQUIRE(BG >= 1 && Qb >= 1 && Kb >= 1 && Pq >= 1 && Pk >= 1, "invalid score shape");
  SPRUCE_REQUIRE(P >= 4 && P % 4 == 0, "projection dim must be a positive multiple of 4, got %lld", (long long)P);
  SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(qp) % 16 == 0 && reinterpret_cast<uintptr_t>(kp) % 16 == 0,
                 "qp and kp must be 16-byte aligned");
  SPRUCE_REQUIRE(BG < 65536 && Qb < (1 << 30) && Kb < (1 << 30) && Pq * Pk * P < ((int64_t)1 << 30),
                 "score shape out of range");
  SPRUCE_REQUIRE(causal >= 0 && causal <= 2, "causal must be 0, 1 or 2, got %d", causal);
  ScoreParams p{qp, kp, scores, (int)Qb, (int)Kb, (int)Pq, (int)Pk, (int)P, div, causal};
  const int64_t lds = (int64_t)(kTI * Pq * P + kTJ * (Pk * P + 4)) * 4;
  if (lds > 160 * 1024) {
    const int64_t total = BG * Qb * Kb;
    const int64_t blocks = (total + 255) / 256;
    SPRUCE_REQUIRE(blocks < ((int64_t)1 << 31), "score matrix too large");
    hipLaunchKernelGGL(gate_scores_direct_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p,
                       total);
    return check_launch("gate_scores_direct_kernel");
  }
  const bool tri = causal == 2 && Qb == Kb;
  if (!tri && causal == 2) p.causal = 1;
  if (Pq == 1 && (Pk == 1 || Pk == 2) && P % kGS == 0 && reinterpret_cast<uintptr_t>(scores) % 16 == 0) {
    // 32-query-block tiles: twice as many workgroups as 64-block tiles,
    // which evens out the per-CU share of a few hundred tiles.
    constexpr int TR = kScoreTR, R = 16 * TR;
    const int64_t nt = (Qb + kGT - 1) / kGT;
    const int64_t ntri = (kGT / R) * (nt * (nt + 1) / 2);
    SPRUCE_REQUIRE(!tri || BG * ntri < ((int64_t)1 << 31), "score matrix too large");
    const dim3 grid = tri ? dim3((unsigned)(BG * ntri))
                          : dim3((unsigned)((Qb + R - 1) / R), (unsigned)((Kb + kGT - 1) / kGT), (unsigned)BG);
    if (Pk == 1)
      hipLaunchKernelGGL((gate_scores_tile_kernel<1, TR>), grid, dim3(256), 0, (hipStream_t)stream, p);
    else
      hipLaunchKernelGGL((gate_scores_tile_kernel<2, TR>), grid, dim3(256), 0, (hipStream_t)stream, p);
    return check_launch("gate_scores_tile_kernel");
  }
  const dim3 grid((unsigned)((Qb + kTI - 1) / kTI), (unsigned)((Kb + kTJ - 1) / kTJ), (unsigned)BG);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute((const void*)gate_scores_kernel,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error((int)e, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(gate_scores_kernel, grid, dim3(256), (size_t)lds, (hipStream_t)stream, p);
  return check_launch("gate_scores_kernel");
}

extern "C" int spruce_causal_topk(const float* scores, int64_t R, int64_t Qb, int64_t Kb, int64_t k, int32_t* out,
                                  void* stream) {
  SPRUCE_REQUIRE(scores && out, "scores and out must be non-null");
  SPRUCE_REQUIRE(R >= 1 && Qb >= 1 && Kb >= 1 && k >= 1, "invalid top-k shape");
  SPRUCE_REQUIRE(Kb <= kTopkMaxKb, "at most %d key blocks per row are supported, got %lld", kTopkMaxKb,
                 (long long)Kb);
  SPRUCE_REQUIRE(R * Qb < ((int64_t)1 << 31), "too many rows");
  if (Kb <= kWaveTopkKb) {
    const int64_t rows = R * Qb;
    hipLaunchKernelGGL(causal_topk_wave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, scores, rows, (int)Qb, (int)Kb, (int)k, out);
    return check_launch("causal_topk_wave_kernel");
  }
  hipLaunchKernelGGL(causal_topk_kernel, dim3((unsigned)(R * Qb)), dim3(256), 0, (hipStream_t)stream, scores,
                     (int)Qb, (int)Kb, (int)k, out);
  return check_launch("causal_topk_kernel");
}

extern "C" int spruce_select_flat_supported(int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype, int64_t P) {
  if (Hkv < 1 || Hq < Hkv || Hq % Hkv != 0 || T < 1) return 0;
  const int64_t nb = (T + kSelBlock - 1) / kSelBlock;
  return D == kFD && P == kFP && Hq / Hkv <= kPoolMaxG && nb <= kWaveTopkKb &&
         (dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16);
}

extern "C" int64_t spruce_select_flat_workspace_bytes(int64_t B, int64_t Hkv, int64_t T, int64_t P) {
  if (B < 1 || Hkv < 1 || T < 1 || P < 1) return -1;
  return B * Hkv * 2 * P * ((T + kSelBlock - 1) / kSelBlock) * (int64_t)sizeof(float);
}

extern "C" int spruce_select_flat(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4], int64_t B,
                                  int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype, const float* wq,
                                  const float* wk, int64_t P, float div, int64_t top_k, void* workspace,
                                  int64_t workspace_bytes, int32_t* out, void* stream) {
  SPRUCE_REQUIRE(q && qs && k && ks && wq && wk && out && workspace, "q, k, weights, workspace and out must be non-null");
  SPRUCE_REQUIRE(B >= 1 && T >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "invalid shape");
  SPRUCE_REQUIRE(B * Hkv < (1 << 20) && T < (1 << 30), "shape out of range");
  SPRUCE_REQUIRE(spruce_select_flat_supported(Hq, Hkv, T, D, dtype, P),
                 "fused selector needs head_dim %d, projection dim %d, a 16-bit dtype, at most %d query heads per KV "
                 "head and at most %d key blocks (got D %lld, P %lld, dtype %d, G %lld, T %lld)",
                 kFD, kFP, kPoolMaxG, kWaveTopkKb, (long long)D, (long long)P, dtype, (long long)(Hq / Hkv),
                 (long long)T);
  SPRUCE_REQUIRE(top_k >= 1 && top_k <= (1 << 20), "top_k must be >= 1, got %lld", (long long)top_k);
  SPRUCE_REQUIRE(qs[3] == 1 && ks[3] == 1, "q and k need a contiguous last dim");
  SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && qs[0] % 8 == 0 && qs[1] % 8 == 0 && qs[2] % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(k) % 16 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 && ks[2] % 8 == 0,
                 "q and k rows must be 16-byte aligned");
  SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "workspace must be 16-byte aligned");
  const int64_t need = spruce_select_flat_workspace_bytes(B, Hkv, T, P);
  SPRUCE_REQUIRE(workspace_bytes >= need, "workspace too small: %lld bytes, need %lld", (long long)workspace_bytes,
                 (long long)need);
  const int nb = (int)((T + kSelBlock - 1) / kSelBlock);
  const int BG = (int)(B * Hkv);
  SelKeysParams kp{};
  kp.k = k;
  for (int i = 0; i < 4; ++i) kp.ks[i] = ks[i];
  kp.wk = wk;
  kp.kp4 = static_cast<float*>(workspace);
  kp.Hkv = (int)Hkv;
  kp.T = (int)T;
  kp.nb = nb;
  kp.tiles = (nb + kKeyBlocks - 1) / kKeyBlocks;
  const int64_t kgrid = (int64_t)BG * kp.tiles;
  SPRUCE_REQUIRE(kgrid < ((int64_t)1 << 31), "grid too large");
  if (dtype == SPRUCE_DTYPE_BF16)
    hipLaunchKernelGGL(select_keys_kernel<InBF16>, dim3((unsigned)kgrid), dim3(256), 0, (hipStream_t)stream, kp);
  else
    hipLaunchKernelGGL(select_keys_kernel<InF16>, dim3((unsigned)kgrid), dim3(256), 0, (hipStream_t)stream, kp);
  int rc = check_launch("select_keys_kernel");
  if (rc != SPRUCE_OK) return rc;

  SelRowsParams rp{};
  rp.q = q;
  for (int i = 0; i < 4; ++i) rp.qs[i] = qs[i];
  rp.wq = wq;
  rp.kp4 = static_cast<const float*>(workspace);
  rp.out = out;
  rp.Hkv = (int)Hkv;
  rp.T = (int)T;
  rp.nb = nb;
  rp.k = (int)top_k;
  rp.BG = BG;
  rp.row_tiles = (nb + kFRows - 1) / kFRows;
  const int64_t ntiles = (int64_t)BG * rp.row_tiles;
  SPRUCE_REQUIRE(ntiles < ((int64_t)1 << 30), "too many row tiles");
  rp.ntiles = (int)ntiles;
  rp.div = div;
  const int64_t G = Hq / Hkv;
  const int64_t slice = ((T - 1) * qs[2] + (G - 1) * qs[1] + D) * 2;
  SPRUCE_REQUIRE(qs[1] >= 0 && qs[2] >= 0 && slice < ((int64_t)1 << 31) && (G - 1) * qs[1] * 2 < ((int64_t)1 << 31),
                 "fused selector needs each (batch, KV group) slice of q within 2^31 bytes (got %lld)",
                 (long long)slice);
  rp.slice_bytes = (int)slice;
  // One persistent workgroup per CU (each holds 8 waves), at most one per tile.
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return set_error((int)e, "device query failed: %s", hipGetErrorString(e));
  const int grid = (int)(ntiles < cus ? ntiles : cus);
  const bool bf = dtype == SPRUCE_DTYPE_BF16;
  const dim3 g3((unsigned)grid), b3(512);
  hipStream_t st = (hipStream_t)stream;
  switch (Hq / Hkv) {
#define SPRUCE_ROWS_CASE(GG)                                                                            \
  case GG:                                                                                              \
    if (bf) hipLaunchKernelGGL((select_rows_kernel<InBF16, GG>), g3, b3, 0, st, rp);                    \
    else hipLaunchKernelGGL((select_rows_kernel<InF16, GG>), g3, b3, 0, st, rp);                        \
    break;
    SPRUCE_ROWS_CASE(1)
    SPRUCE_ROWS_CASE(2)
    SPRUCE_ROWS_CASE(3)
    SPRUCE_ROWS_CASE(4)
    SPRUCE_ROWS_CASE(5)
    SPRUCE_ROWS_CASE(6)
    SPRUCE_ROWS_CASE(7)
    SPRUCE_ROWS_CASE(8)
#undef SPRUCE_ROWS_CASE
    default:
      return set_error(SPRUCE_EINVAL, "unsupported query heads per KV head: %lld", (long long)(Hq / Hkv));
  }
  return check_launch("select_rows_kernel");
}

extern "C" int spruce_selector_pool_project(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                            int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, int dtype,
                                            const float* wq, const float* wk, int64_t P, float* qp, float* kp,
                                            void* stream) {
  SPRUCE_REQUIRE(q && qs && k && ks && wq && wk && qp && kp, "q, k, weights and outputs must be non-null");
  SPRUCE_REQUIRE(B >= 1 && T >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "invalid shape");
  SPRUCE_REQUIRE(D == kFD && P == kFP && Hq / Hkv <= kPoolMaxG &&
                     (dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16),
                 "pooled projection needs head_dim %d, projection dim %d, a 16-bit dtype and at most %d query "
                 "heads per KV head (got D %lld, P %lld, dtype %d, G %lld)",
                 kFD, kFP, kPoolMaxG, (long long)D, (long long)P, dtype, (long long)(Hq / Hkv));
  SPRUCE_REQUIRE(qs[3] == 1 && ks[3] == 1, "q and k need a contiguous last dim");
  SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && qs[0] % 8 == 0 && qs[1] % 8 == 0 && qs[2] % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(k) % 16 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 && ks[2] % 8 == 0,
                 "q and k rows must be 16-byte aligned");
  const int64_t G = Hq / Hkv;
  const int64_t qslice = ((T - 1) * qs[2] + (G - 1) * qs[1] + D) * 2;
  const int64_t kslice = ((T - 1) * ks[2] + D) * 2;
  SPRUCE_REQUIRE(qs[1] >= 0 && qs[2] >= 0 && ks[2] >= 0 && qslice < ((int64_t)1 << 31) &&
                     kslice < ((int64_t)1 << 31),
                 "pooled projection needs each (batch, KV group) slice of q and k within 2^31 bytes");
  const int64_t nb = (T + kSelBlock - 1) / kSelBlock;
  const int64_t ntasks = B * Hkv * nb;
  SPRUCE_REQUIRE(ntasks < ((int64_t)1 << 30), "too many blocks");
  PoolProjParams pp{};
  pp.q = q;
  pp.k = k;
  for (int i = 0; i < 4; ++i) {
    pp.qs[i] = qs[i];
    pp.ks[i] = ks[i];
  }
  pp.wq = wq;
  pp.wk = wk;
  pp.qp = qp;
  pp.kp = kp;
  pp.Hkv = (int)Hkv;
  pp.T = (int)T;
  pp.nb = (int)nb;
  pp.BG = (int)(B * Hkv);
  pp.ntasks = (int)ntasks;
  pp.qslice = (int)qslice;
  pp.kslice = (int)kslice;
  // One persistent workgroup of 8 wavefronts per CU (the weights fill 128 KB of LDS).
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return set_error((int)e, "device query failed: %s", hipGetErrorString(e));
  const int64_t need = (ntasks + 7) / 8;
  const int grid = (int)(need < cus ? need : cus);
  const bool bf = dtype == SPRUCE_DTYPE_BF16;
  const dim3 g3((unsigned)grid), b3(512);
  hipStream_t st = (hipStream_t)stream;
  switch (G) {
#define SPRUCE_PP_CASE(GG)                                                                \
  case GG:                                                                                \
    if (bf) hipLaunchKernelGGL((pool_project_kernel<InBF16, GG>), g3, b3, 0, st, pp);     \
    else hipLaunchKernelGGL((pool_project_kernel<InF16, GG>), g3, b3, 0, st, pp);         \
    break;
    SPRUCE_PP_CASE(1)
    SPRUCE_PP_CASE(2)
    SPRUCE_PP_CASE(3)
    SPRUCE_PP_CASE(4)
    SPRUCE_PP_CASE(5)
    SPRUCE_PP_CASE(6)
    SPRUCE_PP_CASE(7)
    SPRUCE_PP_CASE(8)
#undef SPRUCE_PP_CASE
    default:
      return set_error(SPRUCE_EINVAL, "unsupported query heads per KV head: %lld", (long long)G);
  }
  return check_launch("pool_project_kernel");
}
