// Selector prototype features, in the model dtype:
//
//   group_avg   _group_avg_tokens (teacher/chunked_extract.py:75-80): the H/G
//               query heads of each KV group averaged per token.
//   proto_pool  _proto_pool_seq (teacher/chunked_extract.py:27-72) fused with
//               the group average: per block of `block` tokens, prototype 0 is
//               the mean over the block's real rows and prototypes 1..k
//               (k = min(P-1, block)) are the k rows farthest from it in
//               float32 squared L2, farthest first; slots past the real rows
//               hold the mean.
//
// Arithmetic (compiled without contraction, IEEE division):
//   group average  rnd(sum_h x_h * fl(1/rep)), heads summed in order from 0.0f
//                  (torch's GPU mean: float accumulation times the factor
//                  1/n); rep == 1 copies the row unchanged.
//   block mean     rnd(rnd(sum_t a_t) / n), tokens summed in order (the
//                  reference sums in the model dtype, then divides in it).
//   distance       sum_d (a_d - m_d)^2 in float32, dims in order.
//   top-k          descending distance, ties to the lower row, NaN largest.
// rnd() rounds to the model dtype (nearest even); float32 input is exact.
// One workgroup per (batch, KV group, block); the block tile is held in LDS,
// as float, or for 16-bit single-head input (the key side) as the raw 16-bit
// words, which halves the workgroup's LDS.  HBM-bound: every input element is
// read once.
#include <type_traits>

#include "common.h"

namespace spruce {
namespace {

constexpr int kProtoMaxD = 128;
constexpr int kProtoMaxBlock = 64;
constexpr int kProtoMaxP = 65;

struct ProtoParams {
  const void* x;
  int64_t xs[4];
  int B, H, G, L, D, block, P, nb, dtype, rep;
  float inv_rep;
  void* out;  // [B, G, nb, P, D] in x's dtype, contiguous
};

__device__ __forceinline__ float round_to(float v, int dtype) {
  if (dtype == SPRUCE_DTYPE_BF16) return (float)(__bf16)v;
  if (dtype == SPRUCE_DTYPE_F16) return (float)(_Float16)v;
  return v;
}

__device__ __forceinline__ float load1(const void* base, int64_t elem, int dtype) {
  if (dtype == SPRUCE_DTYPE_F32) return static_cast<const float*>(base)[elem];
  const uint32_t bits = static_cast<const uint16_t*>(base)[elem];
  return dtype == SPRUCE_DTYPE_F16 ? unpack1<true>(bits) : unpack1<false>(bits);
}

__device__ __forceinline__ void store1(void* base, int64_t elem, int dtype, float v) {
  if (dtype == SPRUCE_DTYPE_F32) {
    static_cast<float*>(base)[elem] = v;
  } else if (dtype == SPRUCE_DTYPE_F16) {
    static_cast<_Float16*>(base)[elem] = (_Float16)v;
  } else {
    static_cast<__bf16*>(base)[elem] = (__bf16)v;
  }
}

// Group average of the rep heads starting at head h0 for token t, dims
// [8c, 8c+8) (vector path) -- written to dst[0..8).
__device__ __forceinline__ void group_avg8(const ProtoParams& p, int b, int h0, int t, int c, float* dst) {
  const int64_t e0 = (int64_t)b * p.xs[0] + (int64_t)t * p.xs[2] + 8 * c;
  float s[8];
  if (p.rep > 1 && p.rep <= 8) {
    // Up to 8 heads: every load is issued before the first add, so the row
    // costs one memory round trip; the sum is the same ordered sequence.
    float v[8][8];
#pragma unroll
    for (int h = 0; h < 8; ++h)
      if (h < p.rep) load8f(p.x, e0 + (int64_t)(h0 + h) * p.xs[1], p.dtype, v[h]);
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f + v[0][j];
#pragma unroll
    for (int h = 1; h < 8; ++h)
      if (h < p.rep)
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] = s[j] + v[h][j];
#pragma unroll
    for (int j = 0; j < 8; ++j) dst[j] = round_to(s[j] * p.inv_rep, p.dtype);
    return;
  }
  load8f(p.x, e0 + (int64_t)h0 * p.xs[1], p.dtype, s);
  if (p.rep > 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f + s[j];
    for (int h = 1; h < p.rep; ++h) {
      float v[8];
      load8f(p.x, e0 + (int64_t)(h0 + h) * p.xs[1], p.dtype, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] = s[j] + v[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = round_to(s[j] * p.inv_rep, p.dtype);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) dst[j] = s[j];
}

__device__ __forceinline__ float group_avg1(const ProtoParams& p, int b, int h0, int t, int d) {
  const int64_t e0 = (int64_t)b * p.xs[0] + (int64_t)t * p.xs[2] + (int64_t)d * p.xs[3];
  float s = load1(p.x, e0 + (int64_t)h0 * p.xs[1], p.dtype);
  if (p.rep == 1) return s;
  s = 0.0f + s;
  for (int h = 1; h < p.rep; ++h) s = s + load1(p.x, e0 + (int64_t)(h0 + h) * p.xs[1], p.dtype);
  return round_to(s * p.inv_rep, p.dtype);
}

// Token chunks per thread whose loads are issued together on the key side
// (one head): a 64-token block of D = 128 is 4 chunks per thread.
constexpr int kProtoBatchK = 4;

// Token chunks whose loads are issued together in the 16-bit group average.
// Measured at cfg3 (Q, 28/4 heads, 64K tokens): 0.129 ms with group_avg8,
// 0.097 ms with 2, 0.098 ms with 1, 0.101 ms with 4.
constexpr int kProtoBatch = 2;
// Load paths: kProtoAny (every dtype and layout), kProtoGroup16 (16-bit,
// contiguous rows, 2..8 heads per group), kProtoOne16 (16-bit, contiguous
// rows, one head: the only path with a 16-bit tile).  F16: the 16-bit input
// is f16 (else bf16).  At the key side the 16-bit tile (7 instead of 4
// workgroups per CU) takes cfg3's K 32 -> 26 us; at the group-average path,
// bound by its 7 heads' loads, a 16-bit tile measured the same as this float
// one (91.5 vs 91.2 us).
constexpr int kProtoAny = 0, kProtoGroup16 = 1, kProtoOne16 = 2;

// Rows of the block tile padded by 16 bytes: 16-byte aligned for the vector
// distance reads and spread over the banks.
template <bool T16>
constexpr int proto_tstr() { return kProtoMaxD + (T16 ? 8 : 4); }
constexpr int kProtoTileBytes = kProtoMaxBlock * (kProtoMaxD + 4) * 4;  // the float tile (the larger)

// Raw 16-byte chunks of one head's block (the key side): kProtoBatchK per
// thread cover a 64 x 128 block; chunks past the block load the last one
// again (in range; not stored).
__device__ __forceinline__ void load_block_raw(const ProtoParams& p, int b, int h0, int t0, int n,
                                               uint4 (&raw)[kProtoBatchK]) {
  const int dch = p.D >> 3;
  const int ne = n * dch;
  const uint16_t* xb = static_cast<const uint16_t*>(p.x) + (int64_t)b * p.xs[0] + (int64_t)h0 * p.xs[1];
#pragma unroll
  for (int k = 0; k < kProtoBatchK; ++k) {
    const int e = min((int)threadIdx.x + 256 * k, ne - 1);
    const int t = e / dch, c = e - (e / dch) * dch;
    raw[k] = *reinterpret_cast<const uint4*>(xb + (int64_t)(t0 + t) * p.xs[2] + 8 * c);
  }
}

// One (batch, KV group, block i) of proto_pool_kernel, with the block tile at
// tile_mem (proto_tstr<T16>() elements per row).  With PRE (the one-head
// 16-bit path, a block of at most 256 * kProtoBatchK chunks) the chunks in
// kraw were loaded by load_block_raw and are stored instead of loaded.
template <int PATH, bool F16, bool PRE>
__device__ __forceinline__ void proto_pool_block(const ProtoParams& p, int b, int g, int i, void* tile_mem,
                                                 float* mean, int* pick, const uint4 (&kraw)[kProtoBatchK]) {
  constexpr bool T16 = PATH == kProtoOne16;
  using TileT = std::conditional_t<T16, uint16_t, float>;
  constexpr int TSTR = proto_tstr<T16>();
  TileT (*tile)[TSTR] = reinterpret_cast<TileT (*)[TSTR]>(tile_mem);
  auto tget = [&](int t, int d) -> float {
    if constexpr (T16) {
      return unpack1<F16>(tile[t][d]);
    } else {
      return tile[t][d];
    }
  };
  const int tid = threadIdx.x;
  const int t0 = i * p.block;
  const int n = min(p.block, p.L - t0);
  const int h0 = g * p.rep;
  const bool vec = (p.D & 7) == 0 && p.xs[3] == 1;

  if constexpr (PATH == kProtoGroup16) {
    // 16-bit inputs: the raw 16-byte loads of kProtoBatch token chunks (all
    // their heads) are issued before the first add and widened only when
    // added, so a 64-token block of D = 128 costs 4 / kProtoBatch memory
    // round trips; the sums are the same ordered sequence as group_avg8.
    // The loads are unconditional, so they issue back to back: heads past
    // rep re-read head h0's chunk and chunks past the block re-read its last
    // one (both in range, neither added or stored).
    const int dch = p.D >> 3;
    const int ne = n * dch;  // 16-byte chunks per head of the block, >= 1
    const uint16_t* xb = static_cast<const uint16_t*>(p.x) + (int64_t)b * p.xs[0];
    for (int e0 = tid; e0 < ne; e0 += 256 * kProtoBatch) {
      uint4 raw[kProtoBatch][8];
#pragma unroll
      for (int k = 0; k < kProtoBatch; ++k) {
        const int e = min(e0 + 256 * k, ne - 1);
        const int t = e / dch, c = e - (e / dch) * dch;
        const uint16_t* row = xb + (int64_t)(t0 + t) * p.xs[2] + 8 * c;
#pragma unroll
        for (int h = 0; h < 8; ++h)
          raw[k][h] = *reinterpret_cast<const uint4*>(row + (int64_t)(h0 + (h < p.rep ? h : 0)) * p.xs[1]);
      }
      // Keep every load ahead of the first add (the scheduler otherwise sinks
      // the second chunk's loads to their uses, one round trip each).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < kProtoBatch; ++k) {
        const int e = e0 + 256 * k;
        if (e >= ne) break;
        const int t = e / dch, c = e - (e / dch) * dch;
        float sum[8];
#pragma unroll
        for (int h = 0; h < 8; ++h) {
          if (h >= p.rep) break;
          const uint32_t w[4] = {raw[k][h].x, raw[k][h].y, raw[k][h].z, raw[k][h].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float lo = unpack1<F16>(w[i] & 0xffffu);
            const float hi = unpack1<F16>(w[i] >> 16);
            sum[2 * i] = h == 0 ? 0.0f + lo : sum[2 * i] + lo;
            sum[2 * i + 1] = h == 0 ? 0.0f + hi : sum[2 * i + 1] + hi;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[t][8 * c + j] = round_to(sum[j] * p.inv_rep, p.dtype);
      }
    }
  } else if constexpr (PATH == kProtoOne16) {
    // One head (the key side): the row is copied unchanged, so the raw
    // 16-byte chunks of kProtoBatchK token chunks are all loaded first and
    // then stored into the tile as they are (one memory round trip for a
    // 64 x 128 block).
    const int dch = p.D >> 3;
    const int ne = n * dch;  // 16-byte chunks of the block, >= 1
    const uint16_t* xb = static_cast<const uint16_t*>(p.x) + (int64_t)b * p.xs[0] + (int64_t)h0 * p.xs[1];
    if constexpr (PRE) {
      // Constant indices into kraw, so the chunks stay in registers.
      static_assert(kProtoBatchK == 4, "four preloaded chunks per thread");
      auto put = [&](int k, const uint4 v) __attribute__((always_inline)) {
        const int e = tid + 256 * k;
        if (e < ne) {
          const int t = e / dch, c = e - (e / dch) * dch;
          *reinterpret_cast<uint4*>(&tile[t][8 * c]) = v;
        }
      };
      put(0, kraw[0]);
      put(1, kraw[1]);
      put(2, kraw[2]);
      put(3, kraw[3]);
    }
    for (int e0 = tid; !PRE && e0 < ne; e0 += 256 * kProtoBatchK) {
      // Chunks past the block load the last one again (in range; not stored).
      uint4 raw[kProtoBatchK];
#pragma unroll
      for (int k = 0; k < kProtoBatchK; ++k) {
        const int e = min(e0 + 256 * k, ne - 1);
        const int t = e / dch, c = e - (e / dch) * dch;
        raw[k] = *reinterpret_cast<const uint4*>(xb + (int64_t)(t0 + t) * p.xs[2] + 8 * c);
      }
#pragma unroll
      for (int k = 0; k < kProtoBatchK; ++k) {
        const int e = e0 + 256 * k;
        if (e < ne) {
          const int t = e / dch, c = e - (e / dch) * dch;
          *reinterpret_cast<uint4*>(&tile[t][8 * c]) = raw[k];
        }
      }
    }
  } else if (vec) {
    const int dch = p.D >> 3;
    for (int e = tid; e < n * dch; e += 256) {
      const int t = e / dch, c = e - (e / dch) * dch;
      float v[8];
      group_avg8(p, b, h0, t0 + t, c, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) tile[t][8 * c + j] = v[j];
    }
  } else {
    for (int e = tid; e < n * p.D; e += 256) {
      const int t = e / p.D, d = e - (e / p.D) * p.D;
      tile[t][d] = group_avg1(p, b, h0, t0 + t, d);
    }
  }
  __syncthreads();

  if (tid < p.D) {
    float s = 0.0f;
#pragma unroll 8
    for (int t = 0; t < n; ++t) s = s + tget(t, tid);
    mean[tid] = round_to(round_to(s, p.dtype) / (float)n, p.dtype);
  }
  __syncthreads();

  const int k = min(p.P - 1, p.block);
  if (tid < 64) {
    // Lane = row of the block; rows past the real ones rank as -inf.
    float dist = -__builtin_inff();
    if (tid < n) {
      float s = 0.0f;
      if ((p.D & 3) == 0) {
#pragma unroll 8
        for (int d = 0; d < p.D; d += 4) {
          float4 x;
          if constexpr (T16) {
            const uint2 w = *reinterpret_cast<const uint2*>(&tile[tid][d]);
            x = float4{unpack1<F16>(w.x & 0xffffu), unpack1<F16>(w.x >> 16), unpack1<F16>(w.y & 0xffffu),
                       unpack1<F16>(w.y >> 16)};
          } else {
            x = *reinterpret_cast<const float4*>(&tile[tid][d]);
          }
          const float4 m = *reinterpret_cast<const float4*>(&mean[d]);
          float diff = x.x - m.x;
          s = s + diff * diff;
          diff = x.y - m.y;
          s = s + diff * diff;
          diff = x.z - m.z;
          s = s + diff * diff;
          diff = x.w - m.w;
          s = s + diff * diff;
        }
      } else {
        for (int d = 0; d < p.D; ++d) {
          const float diff = tget(tid, d) - mean[d];
          s = s + diff * diff;
        }
      }
      dist = s;
    }
    const bool in_block = tid < p.block;
    const uint32_t u = __builtin_bit_cast(uint32_t, dist);
    const uint32_t okey = dist != dist ? 0xffffffffu                    // any NaN ranks above +inf
                                       : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
    bool taken = !in_block;
    // Each round: the largest order key among the rows not yet taken (every
    // such key is at least 0x007fffff, taken rows count as 0), then the
    // lowest row holding it (ties to the lower row).
    for (int j = 0; j < k; ++j) {
      const uint32_t key = taken ? 0u : okey;
      const uint32_t top = wave_max_u32(key);
      const int best = (int)__builtin_ctzll(__ballot(key == top));
      if (tid == best) taken = true;
      if (tid == 0) pick[j] = best;
    }
  }
  __syncthreads();

  const int64_t obase = (((int64_t)b * p.G + g) * p.nb + i) * (int64_t)p.P * p.D;
  for (int e = tid; e < p.P * p.D; e += 256) {
    const int pr = e / p.D, d = e - (e / p.D) * p.D;
    float v = mean[d];
    if (pr >= 1 && pr <= k) {
      const int row = pick[pr - 1];
      if (row < n) v = tget(row, d);
    }
    store1(p.out, obase + e, p.dtype, v);
  }
}

template <int PATH, bool F16>
__global__ __launch_bounds__(256) void proto_pool_kernel(ProtoParams p) {
  constexpr bool T16 = PATH == kProtoOne16;
  __shared__ __attribute__((aligned(16))) char tile[kProtoMaxBlock * proto_tstr<T16>() * (T16 ? 2 : 4)];
  __shared__ __attribute__((aligned(16))) float mean[kProtoMaxD];
  __shared__ int pick[kProtoMaxP];
  const int i = blockIdx.x % p.nb;
  const int bg = blockIdx.x / p.nb;
  const uint4 none[kProtoBatchK] = {};
  proto_pool_block<PATH, F16, false>(p, bg / p.G, bg % p.G, i, tile, mean, pick, none);
}

// Query and key prototypes of the same (batch, KV group, block) in one
// workgroup: the key block's raw loads are issued first and held in
// registers while the query heads are averaged and pooled; then the key
// block is pooled in the same LDS (its 16-bit tile over the dead float one).
// Outputs equal proto_pool_kernel's on each side.
template <int QPATH, bool F16>
__global__ __launch_bounds__(256) void proto_pool_qk_kernel(ProtoParams pq, ProtoParams pk) {
  __shared__ __attribute__((aligned(16))) char tile[kProtoTileBytes];
  __shared__ __attribute__((aligned(16))) float mean[kProtoMaxD];
  __shared__ int pick[kProtoMaxP];
  const int i = blockIdx.x % pq.nb;
  const int bg = blockIdx.x / pq.nb;
  const int b = bg / pq.G, g = bg % pq.G;
  const int t0 = i * pk.block;
  const int n = min(pk.block, pk.L - t0);
  uint4 kraw[kProtoBatchK];
  load_block_raw(pk, b, g, t0, n, kraw);
  const uint4 none[kProtoBatchK] = {};
  proto_pool_block<QPATH, F16, false>(pq, b, g, i, tile, mean, pick, none);
  __syncthreads();  // the query output has read the tile and the mean
  proto_pool_block<kProtoOne16, F16, true>(pk, b, g, i, tile, mean, pick, kraw);
}

__global__ __launch_bounds__(256) void group_avg_kernel(ProtoParams p, int64_t total8) {
  // One thread per (b, g, t, 8-dim chunk) -- vector path only.
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total8) return;
  const int dch = p.D >> 3;
  const int c = (int)(e % dch);
  const int64_t r = e / dch;
  const int t = (int)(r % p.L);
  const int bg = (int)(r / p.L);
  const int g = bg % p.G, b = bg / p.G;
  float v[8];
  group_avg8(p, b, g * p.rep, t, c, v);
  const int64_t o = r * p.D + 8 * c;
#pragma unroll
  for (int j = 0; j < 8; ++j) store1(p.out, o + j, p.dtype, v[j]);
}

__global__ __launch_bounds__(256) void group_avg_scalar_kernel(ProtoParams p, int64_t total) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const int d = (int)(e % p.D);
  const int64_t r = e / p.D;
  const int t = (int)(r % p.L);
  const int bg = (int)(r / p.L);
  const int g = bg % p.G, b = bg / p.G;
  store1(p.out, e, p.dtype, group_avg1(p, b, g * p.rep, t, d));
}

int fill_params(ProtoParams& p, const void* x, const int64_t xs[4], int64_t B, int64_t H, int64_t L, int64_t D,
                int64_t G, int dtype, void* out) {
  SPRUCE_REQUIRE(x && xs && out, "x, strides and out must be non-null");
  SPRUCE_REQUIRE(dtype == SPRUCE_DTYPE_BF16 || dtype == SPRUCE_DTYPE_F16 || dtype == SPRUCE_DTYPE_F32,
                 "unsupported dtype code %d", dtype);
  SPRUCE_REQUIRE(B >= 1 && H >= 1 && L >= 1 && D >= 1 && G >= 1, "invalid shape");
  SPRUCE_REQUIRE(H % G == 0, "H=%lld not divisible by G=%lld", (long long)H, (long long)G);
  SPRUCE_REQUIRE(B < (1 << 20) && H < (1 << 16) && L < ((int64_t)1 << 30), "shape out of range");
  for (int i = 0; i < 4; ++i) SPRUCE_REQUIRE(xs[i] >= 0, "negative strides are not supported");
  const int eb = dtype == SPRUCE_DTYPE_F32 ? 4 : 2;
  if ((D & 7) == 0 && xs[3] == 1) {
    SPRUCE_REQUIRE(((uintptr_t)x & 15) == 0 && (xs[0] * eb) % 16 == 0 && (xs[1] * eb) % 16 == 0 &&
                       (xs[2] * eb) % 16 == 0,
                   "x with a contiguous last dim must be 16-byte aligned in every row");
  }
  p.x = x;
  for (int i = 0; i < 4; ++i) p.xs[i] = xs[i];
  p.B = (int)B; p.H = (int)H; p.G = (int)G; p.L = (int)L; p.D = (int)D;
  p.dtype = dtype;
  p.rep = (int)(H / G);
  p.inv_rep = 1.0f / (float)p.rep;
  p.out = out;
  return SPRUCE_OK;
}

}  // namespace
}  // namespace spruce

using namespace spruce;

extern "C" int spruce_proto_pool(const void* x, const int64_t xs[4], int64_t B, int64_t H, int64_t L, int64_t D,
                                 int64_t G, int64_t block, int64_t P, int dtype, void* out, void* stream) {
  ProtoParams p;
  const int rc = fill_params(p, x, xs, B, H, L, D, G, dtype, out);
  if (rc) return rc;
  SPRUCE_REQUIRE(D <= kProtoMaxD, "head_dim must be <= %d, got %lld", kProtoMaxD, (long long)D);
  SPRUCE_REQUIRE(block >= 1 && block <= kProtoMaxBlock, "block must be in [1, %d], got %lld", kProtoMaxBlock,
                 (long long)block);
  SPRUCE_REQUIRE(P >= 1 && P <= kProtoMaxP, "P must be in [1, %d], got %lld", kProtoMaxP, (long long)P);
  p.block = (int)block;
  p.P = (int)P;
  p.nb = (int)((L + block - 1) / block);
  const int64_t grid = B * G * (int64_t)p.nb;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "too many blocks");
  const bool vec16 = (D & 7) == 0 && xs[3] == 1 && dtype != SPRUCE_DTYPE_F32;
  const bool f16 = dtype == SPRUCE_DTYPE_F16;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, p);
  };
  if (vec16 && p.rep == 1)
    f16 ? launch(proto_pool_kernel<kProtoOne16, true>) : launch(proto_pool_kernel<kProtoOne16, false>);
  else if (vec16 && p.rep <= 8)
    f16 ? launch(proto_pool_kernel<kProtoGroup16, true>) : launch(proto_pool_kernel<kProtoGroup16, false>);
  else
    launch(proto_pool_kernel<kProtoAny, false>);
  return check_launch("proto_pool_kernel");
}

extern "C" int spruce_group_avg_tokens(const void* x, const int64_t xs[4], int64_t B, int64_t H, int64_t L,
                                       int64_t D, int64_t G, int dtype, void* out, void* stream) {
  ProtoParams p;
  const int rc = fill_params(p, x, xs, B, H, L, D, G, dtype, out);
  if (rc) return rc;
  p.block = 1; p.P = 1; p.nb = 0;
  if ((D & 7) == 0 && xs[3] == 1) {
    const int64_t total8 = B * G * L * (D / 8);
    SPRUCE_REQUIRE((total8 + 255) / 256 < ((int64_t)1 << 31), "tensor too large");
    hipLaunchKernelGGL(group_avg_kernel, dim3((unsigned)((total8 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, p, total8);
  } else {
    const int64_t total = B * G * L * D;
    SPRUCE_REQUIRE((total + 255) / 256 < ((int64_t)1 << 31), "tensor too large");
    hipLaunchKernelGGL(group_avg_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, p, total);
  }
  return check_launch("group_avg_kernel");
}

extern "C" int spruce_proto_pool_qk(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                    int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D, int64_t block,
                                    int64_t P, int dtype, void* out_q, void* out_k, void* stream) {
  ProtoParams pq, pk;
  int rc = fill_params(pq, q, qs, B, Hq, L, D, Hkv, dtype, out_q);
  if (rc) return rc;
  rc = fill_params(pk, k, ks, B, Hkv, L, D, Hkv, dtype, out_k);
  if (rc) return rc;
  SPRUCE_REQUIRE(dtype != SPRUCE_DTYPE_F32 && D % 8 == 0 && D <= kProtoMaxD && qs[3] == 1 && ks[3] == 1 &&
                     pq.rep <= 8,
                 "fused query/key prototypes need 16-bit inputs with a contiguous last dim, head_dim a multiple "
                 "of 8 up to %d and at most 8 query heads per KV head",
                 kProtoMaxD);
  SPRUCE_REQUIRE(block >= 1 && block <= kProtoMaxBlock, "block must be in [1, %d], got %lld", kProtoMaxBlock,
                 (long long)block);
  SPRUCE_REQUIRE(P >= 1 && P <= kProtoMaxP, "P must be in [1, %d], got %lld", kProtoMaxP, (long long)P);
  pq.block = pk.block = (int)block;
  pq.P = pk.P = (int)P;
  pq.nb = pk.nb = (int)((L + block - 1) / block);
  const int64_t grid = B * Hkv * (int64_t)pq.nb;
  SPRUCE_REQUIRE(grid < ((int64_t)1 << 31), "too many blocks");
  const bool f16 = dtype == SPRUCE_DTYPE_F16;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, pq, pk);
  };
  if (pq.rep == 1)
    f16 ? launch(proto_pool_qk_kernel<kProtoOne16, true>) : launch(proto_pool_qk_kernel<kProtoOne16, false>);
  else
    f16 ? launch(proto_pool_qk_kernel<kProtoGroup16, true>) : launch(proto_pool_qk_kernel<kProtoGroup16, false>);
  return check_launch("proto_pool_qk_kernel");
}
