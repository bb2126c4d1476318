// Block-sparse causal GQA prefill forward for gfx950.
//
// Semantics follow the reference PyTorch path sparse/attention.py:186-274 and
// the kernels it stands in for (kernels/seerattention_direct_index_triton.py:
// 27-121, kernels/seerattention_triton.py:18-68): for every query token t of
// query block qb and query head h, softmax(q_t . k_j * scale) over the keys j
// of the selected 64-token key blocks of KV head h / G with j <= t, applied to
// v_j.  Scores and the softmax run in fp32; P is rounded to the MFMA input
// type before P.V, as the reference kernels do (p.to(v.dtype)).
//
// Work decomposition (MI355X-first, not the reference's one-head-per-program):
//   * one workgroup per (batch, KV head, query block, part); the 2G tiles of
//     32 query rows (G query heads x 2 halves of the 64-row block) of that
//     KV head are spread over the parts, one tile per wave;
//   * every selected K/V block is loaded from HBM/L2 once per workgroup into
//     LDS and shared by all of its waves (GQA packing: 7x less K/V traffic than
//     one head per program at Qwen2-7B's 28/4 heads);
//   * S^T = K Q^T on 32x32x16 MFMA puts one query per lane column, so the
//     row max / row sum of the online softmax are per-lane register reductions
//     plus one exchange with lane ^ 32;
//   * O^T = V^T P^T takes P straight from the S^T accumulators as the B
//     operand; V is staged into LDS as it is stored (row-major, like K) and
//     its V^T operands come from gfx950's transposing LDS reads
//     (ds_read_b64_tr_b16, two per operand), picking the keys in the order
//     the accumulator layout hands them out;
//   * K/V staging is double-buffered: the next block's global loads are in
//     flight while the current block is on the matrix cores; one barrier per
//     block.  When a workgroup has a wave without a tile (G = 3, 5, 6, 7 in
//     8-wave workgroups) that wave stages every block alone (the producer
//     form) and the tile waves only compute;
//   * LDS fragment reads are interleaved with the MFMAs that consume them, so
//     the waves' LDS traffic overlaps the matrix cores;
//   * skipped blocks are never touched: the block list is walked once and only
//     listed blocks are loaded.
//
// The dense causal form (every block 0..qb, in order) can also emit the
// selector features of the reference's capture hooks
// (teacher/chunked_extract.py:27-80,163-180) from the tiles it already holds:
// the group-averaged query tokens from each wave's resident Q fragment and the
// key prototypes of block qb from the diagonal K tile left in LDS.
#pragma once

#include <type_traits>

#include "common.h"

namespace spruce {

constexpr int kBlock = 64;

enum : int { kModePadded = 0, kModeCsr = 1, kModeMask = 2, kModeCausal = 3 };

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t qs[4], ks[4], vs[4], os[4];
  int B, Hq, Hkv, T, G, Qb, parts;
  float cs;    // multiplier of raw scores inside exp2 (scale*log2 e, or 1 when Q is prescaled)
  float qmul;  // multiplier applied to Q before rounding when prescaled
  int prescale;
  // padded index list
  const int32_t* idx;
  int64_t is[4];
  int K;
  // CSR list
  const int32_t* indptr;
  const int32_t* indices;
  int nnz;
  const int32_t* row_order;
  // block mask
  const uint8_t* mask;
  int64_t ms[4];
  int mask_per_qhead;
  // key padding (padded-list form only): kvalid[b * kvs + t] != 0 marks a
  // real key token; padding keys get no weight.
  const uint8_t* kvalid;
  int64_t kvs;
  // general 4-D attention mask (padded-list form only,
  // sparse/attention.py:225-229): element strides ams over [B, Hm, Tq, Tk]
  // (the last one 1), Hm = 1 or Hq; dtype bf16 / f16 / f32 (added to the
  // scaled score) or u8 (bool: nonzero attends, zero gives no weight).
  // amask_mul = log2(e) / cs turns a mask value into raw score units;
  // amask_vec: 4-element groups may be read as one aligned load;
  // amask_rows16: 16-byte row pieces may be read (base and row strides
  // 16-byte aligned); amask_tk: the mask's key extent.
  const void* amask;
  int64_t ams[4];
  int amask_dtype, amask_heads, amask_vec, amask_rows16, amask_tk;
  float amask_mul;
  // residual summaries (sparse/attention.py:226-265): per row, nodes
  // [B, Hkv, Qb, S] int32 (-1 = none); table keys/values [B, Hkv, N, P, D]
  // (float32, or already rounded to the MFMA input type when sum16) and
  // natural-log counts [B, N, P] float32, all contiguous.
  const int32_t* snode;
  int64_t sns[4];
  int S, N, P, sum16;
  const void* skey;
  const void* sval;
  const float* slog;
  float sbias;  // log counts -> raw score units: log2(e) / cs
  int tpp;  // tiles per part: waves 0..tpp-1 of a workgroup own a tile
  // feature capture (dense causal form): group-averaged queries
  // [B, Hkv, T, D] and key prototypes [B, Hkv, Qb, P, D], model dtype,
  // contiguous; each part covers tpp / G whole 32-row halves of the block.
  void* qgrp;
  void* kproto;
  float inv_rep;
};

struct F32x8 {
  float4 a, b;
};
template <typename TIn>
using raw8_t = typename std::conditional<TIn::bytes == 2, uint4, F32x8>::type;

template <typename TIn>
__device__ __forceinline__ raw8_t<TIn> raw_load8(const char* p, bool valid) {
  raw8_t<TIn> r{};
  if (valid) r = *reinterpret_cast<const raw8_t<TIn>*>(p);
  return r;
}

template <typename TIn, bool F16>
__device__ __forceinline__ uint4 raw_to_mfma(const raw8_t<TIn>& r) {
  if constexpr (TIn::bytes == 2) {
    return r;
  } else {
    return uint4{pack2<F16>(r.a.x, r.a.y), pack2<F16>(r.a.z, r.a.w),
                 pack2<F16>(r.b.x, r.b.y), pack2<F16>(r.b.z, r.b.w)};
  }
}

__device__ __forceinline__ uint32_t elem16(const uint4& r, int e) {
  const uint32_t w = (e >> 1) == 0 ? r.x : (e >> 1) == 1 ? r.y : (e >> 1) == 2 ? r.z : r.w;
  return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

// V^T operand from a row-major V tile ([key][d], 16-bit elements) by the
// gfx950 transposing LDS read: within each 16-lane group, result lane i
// element j is element i % 4 of the 4 consecutive values that source lane
// i / 4 + 4 j points at.  Two reads give a lane the 8 keys of its MFMA
// k-positions for one d.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
// 16 bytes per lane from a buffer straight into LDS: lane l's bytes land at
// lds + 16 l (buffer_load_dwordx4 ... lds, base in M0); out-of-range
// offsets write zeros.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(uint2, r);
}

// ------------------------------------------------------------ block lists
// Each iterator yields the usable key blocks of one (batch, KV head, query
// block) row in list order: ids in [0, qb].  `en` says whether the wave's own
// query head attends the block (only the per-query-head mask can say no).
// All lanes of all waves walk the same sequence.
template <int MODE>
struct BlockIter;

template <>
struct BlockIter<kModePadded> {
  const int32_t* row;
  int64_t stride;
  int n, pos, qb;
  __device__ void init(const AttnParams& p, int b, int g, int qb_, int, int, int, bool) {
    row = p.idx + (int64_t)b * p.is[0] + (int64_t)g * p.is[1] + (int64_t)qb_ * p.is[2];
    stride = p.is[3];
    n = p.K;
    pos = 0;
    qb = qb_;
  }
  __device__ bool next(int& id, bool& en) {
    while (pos < n) {
      const int v = __builtin_amdgcn_readfirstlane(row[(int64_t)pos * stride]);
      ++pos;
      if (v >= 0 && v <= qb) {
        id = v;
        en = true;
        return true;
      }
    }
    return false;
  }
};

template <>
struct BlockIter<kModeCsr> {
  const int32_t* row;
  int n, pos, qb;
  __device__ void init(const AttnParams& p, int b, int g, int qb_, int, int, int, bool) {
    const int64_t r = ((int64_t)b * p.Hkv + g) * p.Qb + qb_;
    int start = __builtin_amdgcn_readfirstlane(p.indptr[r]);
    int end = __builtin_amdgcn_readfirstlane(p.indptr[r + 1]);
    start = start < 0 ? 0 : (start > p.nnz ? p.nnz : start);
    end = end < start ? start : (end > p.nnz ? p.nnz : end);
    row = p.indices + start;
    n = end > start ? end - start : 0;
    pos = 0;
    qb = qb_;
  }
  __device__ bool next(int& id, bool& en) {
    while (pos < n) {
      const int v = __builtin_amdgcn_readfirstlane(row[pos]);
      ++pos;
      if (v >= 0 && v <= qb) {
        id = v;
        en = true;
        return true;
      }
    }
    return false;
  }
};

// Dense causal: every key block 0..qb, in order (the diagonal block last).
template <>
struct BlockIter<kModeCausal> {
  int pos, qb;
  __device__ void init(const AttnParams&, int, int, int qb_, int, int, int, bool) {
    pos = 0;
    qb = qb_;
  }
  __device__ bool next(int& id, bool& en) {
    if (pos > qb) return false;
    id = pos++;
    en = true;
    return true;
  }
};

// Mask rows are scanned 64 columns at a time with ballots; the bytes of the
// next 64 columns are loaded one chunk ahead and kept raw, so the wait for
// them falls where they are used (behind any key block loads issued later).
//
// With a per-query-head mask a workgroup walks the union of the mask rows of
// the query heads its tiles belong to.  Those heads are the tile -> head map
// of the kernel applied to the part's tiles [part * tpp, part * tpp + tpp):
//   * half-major order (tile t = half * G + head): heads t mod G, a run of
//     min(tpp, G) consecutive heads that may wrap past G - 1 to head 0;
//   * head-major order (tile t = 2 * head + half): heads t / 2, a run of at
//     most tpp / 2 + 1 heads that never wraps.
// Both are a start head plus a count (<= 8 for parts of <= 8 tiles).
constexpr int kMaxUnion = 8;

template <>
struct BlockIter<kModeMask> {
  const uint8_t* base;  // mask row qb of query head 0 of the KV group
  int64_t hstride, cstride;
  int hstart, G, nunion, own, qb, chunk, lane;
  uint64_t bits, ownbits;
  uint32_t raw[kMaxUnion];  // prefetched bytes of chunk `chunk` for this lane's column
  __device__ void fetch() {
    const int col = chunk * 64 + lane;
#pragma unroll
    for (int h = 0; h < kMaxUnion; ++h) {
      int hh = hstart + h;
      if (hh >= G) hh -= G;
      raw[h] = (h < nunion && col <= qb) ? base[(int64_t)hh * hstride + (int64_t)col * cstride] : 0u;
    }
  }
  __device__ void init(const AttnParams& p, int b, int g, int qb_, int part, int hq, int lane_, bool half_major) {
    cstride = p.ms[3];
    qb = qb_;
    lane = lane_;
    chunk = 0;
    bits = ownbits = 0;
    if (p.mask_per_qhead) {
      base = p.mask + (int64_t)b * p.ms[0] + (int64_t)(g * p.G) * p.ms[1] + (int64_t)qb_ * p.ms[2];
      hstride = p.ms[1];
      G = p.G;
      const int t0 = part * p.tpp;
      if (half_major) {
        hstart = t0 % p.G;
        nunion = p.tpp < p.G ? p.tpp : p.G;
      } else {
        int t1 = t0 + p.tpp;
        if (t1 > 2 * p.G) t1 = 2 * p.G;
        hstart = t0 >> 1;
        nunion = ((t1 - 1) >> 1) - hstart + 1;
      }
      if (nunion > kMaxUnion) nunion = kMaxUnion;  // not reached: parts hold <= 8 tiles
      // Position of the wave's own head in the run (inactive waves: any).
      own = hq - hstart;
      if (own < 0) own += p.G;
      if (own >= nunion) own = nunion - 1;
    } else {
      base = p.mask + (int64_t)b * p.ms[0] + (int64_t)g * p.ms[1] + (int64_t)qb_ * p.ms[2];
      hstride = 0;
      hstart = 0;
      G = 1;
      nunion = 1;
      own = 0;
    }
    fetch();
  }
  __device__ bool next(int& id, bool& en) {
    while (bits == 0) {
      if (chunk * 64 > qb) return false;
      bool u = false, o = false;
#pragma unroll
      for (int h = 0; h < kMaxUnion; ++h) {
        u |= raw[h] != 0u;
        o |= (h == own) && raw[h] != 0u;
      }
      bits = __ballot(u);
      ownbits = __ballot(o);
      ++chunk;
      fetch();
    }
    const int pz = __builtin_ctzll(bits);
    bits &= bits - 1;
    id = (chunk - 1) * 64 + pz;
    en = (ownbits >> pz) & 1;
    return true;
  }
};

// ------------------------------------------------------------------ kernel
// Buffer descriptors: the block's base is folded into the 48-bit base address
// and num_records bounds the valid bytes, so every load or store beyond the
// sequence end (ragged last block) reads zeros or is dropped by the hardware
// range check -- no per-lane branches, and per-lane offsets stay constant.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kOutOfRange = 0x40000000;  // voffset beyond any num_records used here

template <typename TIn>
__device__ __forceinline__ raw8_t<TIn> buf_load8(__amdgpu_buffer_rsrc_t r, int voff) {
  if constexpr (TIn::bytes == 2) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
  } else {
    F32x8 x;
    x.a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
    x.b = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, 0, 0));
    return x;
  }
}

// Rounds 8 loaded elements to the MFMA type, optionally scaled by `mul` first.
template <typename TIn, bool F16>
__device__ __forceinline__ uint4 to_mfma_scaled(const raw8_t<TIn>& r, float mul, bool scaled) {
  if (!scaled) return raw_to_mfma<TIn, F16>(r);
  float f[8];
  if constexpr (TIn::bytes == 2) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = unpack1<F16>(w[i] & 0xffffu);
      f[2 * i + 1] = unpack1<F16>(w[i] >> 16);
    }
  } else {
    f[0] = r.a.x; f[1] = r.a.y; f[2] = r.a.z; f[3] = r.a.w;
    f[4] = r.b.x; f[5] = r.b.y; f[6] = r.b.z; f[7] = r.b.w;
  }
  return uint4{pack2<F16>(f[0] * mul, f[1] * mul), pack2<F16>(f[2] * mul, f[3] * mul),
               pack2<F16>(f[4] * mul, f[5] * mul), pack2<F16>(f[6] * mul, f[7] * mul)};
}

__device__ __forceinline__ uint32_t word_of(const uint4& r, int k) {
  return k == 0 ? r.x : k == 1 ? r.y : k == 2 ? r.z : r.w;
}

// ------------------------------------------------------------ feature capture
// Arithmetic of the selector features (the same operation sequences as the
// standalone prototype kernels, so the results agree bit for bit; no FP
// contraction here):
//   key prototypes of a block: prototype 0 = rnd(rnd(sum_t k_t) / n) over the
//     block's n real rows (rows summed in order from 0.0f; the reference sums
//     and divides in the model dtype, teacher/chunked_extract.py:46-47);
//     prototypes 1..k, k = min(P-1, 64), are the k rows farthest from it in
//     float32 squared L2 (dims in order from 0.0f), farthest first, ties to
//     the lower row, NaN largest (:55-58); slots without a real row hold the
//     mean (:65-72).
//   group-averaged queries: rnd(sum_h q_h * fl(1/G)) over the G query heads of
//     the KV head, heads in order from 0.0f (torch's mean, :75-80); G == 1
//     copies the row.
// rnd() rounds to the model dtype.
template <bool F16>
__device__ __forceinline__ float model_rnd(float x) {
  if constexpr (F16) return (float)(_Float16)x;
  else return (float)(__bf16)x;
}

// Ks: the block's K tile in LDS (row stride KSTR, raw model-dtype bits);
// scratch: >= (D + 64) * 4 bytes of LDS no other wave touches; n: real rows.
// Called by every thread of the workgroup (it contains barriers).
template <int D, int KSTR, int NTHR, bool F16>
__device__ void capture_key_prototypes(const uint16_t* Ks, float* scratch, int n, int P, uint16_t* dst, int tid) {
#pragma clang fp contract(off)
  float* mean = scratch;
  int* pick = reinterpret_cast<int*>(scratch + D);
  if (tid < D) {
    float s = 0.0f;
    for (int t = 0; t < n; ++t) s = s + unpack1<F16>(Ks[t * KSTR + tid]);
    mean[tid] = model_rnd<F16>(model_rnd<F16>(s) / (float)n);
  }
  __syncthreads();
  const int k = P - 1 < kBlock ? P - 1 : kBlock;
  if (tid < 64) {
    // Lane = row of the block; rows past the real ones rank as -inf.
    float dist = -__builtin_inff();
    if (tid < n) {
      float s = 0.0f;
      for (int d = 0; d < D; ++d) {
        const float diff = unpack1<F16>(Ks[tid * KSTR + d]) - mean[d];
        s = s + diff * diff;
      }
      dist = s;
    }
    // Order key: larger distance first, any NaN above +inf, then lower row.
    const uint32_t u = __builtin_bit_cast(uint32_t, dist);
    const uint32_t okey = dist != dist ? 0xffffffffu : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
    // Each round: the largest key among the rows not yet taken (every such
    // key is at least 0x007fffff, taken rows count as 0), then the lowest row
    // holding it.
    bool taken = false;
    for (int j = 0; j < k; ++j) {
      const uint32_t key = taken ? 0u : okey;
      const uint32_t top = wave_max_u32(key);
      const int best = (int)__builtin_ctzll(__ballot(key == top));
      if (tid == best) taken = true;
      if (tid == 0) pick[j] = best;
    }
  }
  __syncthreads();
  constexpr int CH = D / 8;
  for (int c = tid; c < P * CH; c += NTHR) {
    const int slot = c / CH, d0 = (c - slot * CH) * 8;
    const int row = (slot >= 1 && slot <= k) ? pick[slot - 1] : kBlock;
    uint4 w;
    if (row < n) {
      w = *reinterpret_cast<const uint4*>(Ks + row * KSTR + d0);
    } else {
      w = uint4{pack2<F16>(mean[d0], mean[d0 + 1]), pack2<F16>(mean[d0 + 2], mean[d0 + 3]),
                pack2<F16>(mean[d0 + 4], mean[d0 + 5]), pack2<F16>(mean[d0 + 6], mean[d0 + 7])};
    }
    *reinterpret_cast<uint4*>(dst + (int64_t)slot * D + d0) = w;
  }
}

// qst: slot w = lh * G + h holds the 32 rows of query head h, half lh, of
// this part (row stride RS, raw model-dtype bits).  Writes the nh * 32
// group-averaged rows starting at token t_first (rows at or past T skipped).
template <int D, int NTHR, bool F16>
__device__ void capture_group_average(const uint16_t* qst, int RS, int G, int nh, float inv_rep, int t_first, int T,
                                      uint16_t* dst, int tid) {
#pragma clang fp contract(off)
  constexpr int CH = D / 8;
  for (int task = tid; task < nh * 32 * CH; task += NTHR) {
    const int r = task / CH, c = task - (task / CH) * CH;
    if (t_first + r >= T) continue;
    const int lh = r >> 5, rr = r & 31;
    const uint16_t* src = qst + (lh * G * 32 + rr) * RS + 8 * c;
    uint4 w = *reinterpret_cast<const uint4*>(src);
    if (G > 1) {
      float s[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] = 0.0f + unpack1<F16>(elem16(w, j));
      for (int h = 1; h < G; ++h) {
        const uint4 x = *reinterpret_cast<const uint4*>(src + h * 32 * RS);
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] = s[j] + unpack1<F16>(elem16(x, j));
      }
      w = uint4{pack2<F16>(s[0] * inv_rep, s[1] * inv_rep), pack2<F16>(s[2] * inv_rep, s[3] * inv_rep),
                pack2<F16>(s[4] * inv_rep, s[5] * inv_rep), pack2<F16>(s[6] * inv_rep, s[7] * inv_rep)};
    }
    *reinterpret_cast<uint4*>(dst + (int64_t)r * D + 8 * c) = w;
  }
}

// Softmax reference point: the running max is only raised when a row's max
// grows by more than this (log2 units), so most blocks skip the O rescale.
// Exponents stay <= 2^8, far inside fp32/bf16/f16 range; the final O / l is
// unchanged because O and l share the same reference point.
constexpr float kRescaleThreshold = 8.0f;

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x8;
constexpr int kSchedDsRead = 0x100;
// LDS fragment reads in flight ahead of the MFMA that consumes them, in
// K k-steps (two reads each; the V^T loop keeps the same number of reads).
constexpr int kLookahead = 2;

// Four mask values of one row at element el (keys el .. el + 3, of which the
// first nvalid exist) as raw bits, converted only when the scores need them
// (amask_unpack4), so the loads can be issued a block ahead: f32 in w[0..3],
// 16-bit in w[0..1] (element t in half t%2 of w[t/2]), bytes in w[0].
// Missing elements read as zero bits.
__device__ __forceinline__ uint4 amask_fetch4(const AttnParams& p, int64_t el, int nvalid) {
  const int dt = p.amask_dtype;
  if (p.amask_vec && nvalid >= 4) {
    if (dt == SPRUCE_DTYPE_F32) return *reinterpret_cast<const uint4*>(static_cast<const float*>(p.amask) + el);
    if (dt == SPRUCE_DTYPE_U8) {
      return uint4{*reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.amask) + el), 0u, 0u, 0u};
    }
    const uint2 x = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.amask) + el);
    return uint4{x.x, x.y, 0u, 0u};
  }
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (t < nvalid) {
      if (dt == SPRUCE_DTYPE_F32) {
        w[t] = static_cast<const uint32_t*>(p.amask)[el + t];
      } else if (dt == SPRUCE_DTYPE_U8) {
        w[0] |= (uint32_t)static_cast<const uint8_t*>(p.amask)[el + t] << (8 * t);
      } else {
        w[t >> 1] |= (uint32_t)static_cast<const uint16_t*>(p.amask)[el + t] << (16 * (t & 1));
      }
    }
  }
  return uint4{w[0], w[1], w[2], w[3]};
}

// The four values of amask_fetch4 as float: bool masks give 0 (attend) or -inf.
__device__ __forceinline__ void amask_unpack4(int dt, const uint4& x, float (&v)[4]) {
  if (dt == SPRUCE_DTYPE_F32) {
    v[0] = __builtin_bit_cast(float, x.x); v[1] = __builtin_bit_cast(float, x.y);
    v[2] = __builtin_bit_cast(float, x.z); v[3] = __builtin_bit_cast(float, x.w);
  } else if (dt == SPRUCE_DTYPE_U8) {
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = ((x.x >> (8 * t)) & 0xffu) ? 0.f : -INFINITY;
  } else {
    const bool f16 = dt == SPRUCE_DTYPE_F16;
    v[0] = f16 ? unpack1<true>(x.x & 0xffffu) : unpack1<false>(x.x & 0xffffu);
    v[1] = f16 ? unpack1<true>(x.x >> 16) : unpack1<false>(x.x >> 16);
    v[2] = f16 ? unpack1<true>(x.y & 0xffffu) : unpack1<false>(x.y & 0xffffu);
    v[3] = f16 ? unpack1<true>(x.y >> 16) : unpack1<false>(x.y >> 16);
  }
}

template <int D, int WAVES, typename TIn, bool F16, int MODE, bool SUMM = false, bool CAP = false, bool PROD = false,
          bool KVAL = false, bool AMASK = false>
__global__ __launch_bounds__(WAVES * 64) void sparse_prefill_kernel(const AttnParams p) {
  static_assert(!CAP || (MODE == kModeCausal && !SUMM && TIn::bytes == 2),
                "feature capture runs on the dense causal form in the model dtype");
  static_assert(!KVAL || MODE == kModePadded, "key padding is supported for padded block lists");
  static_assert(!AMASK || (MODE == kModePadded && !SUMM && !KVAL && !CAP),
                "the general attention mask is supported for padded block lists without summaries");
  static_assert(!PROD || TIn::bytes == 2, "the producer form stages 16-bit K/V");
  constexpr int NTHR = WAVES * 64;
  constexpr int KSTR = D + 8;        // K tile row stride, 16-bit elements (16 B pad)
  // V tile row stride: rows start 16 banks apart, so the 8 rows x 64 bytes
  // a transposing read touches fall in distinct banks per half-wave.
  constexpr int VSTR = D + 32;
  constexpr int KTILE = kBlock * KSTR;
  constexpr int VTILE = kBlock * VSTR;
  constexpr int BUF = KTILE + VTILE;
  constexpr int KROWCH = D / 8;                  // 8-element chunks per K row
  constexpr int KCHUNKS = kBlock * KROWCH;
  constexpr int KCH = (KCHUNKS + NTHR - 1) / NTHR;
  constexpr int DT = D / 32;  // 32-row tiles of O^T
  constexpr int KS = D / 16;  // k-steps of S^T
  constexpr int EB = TIn::bytes;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps per-wave addresses scalar
  const int l32 = lane & 31, hl = lane >> 5;

  // ---- work item.  Workgroups go round-robin to the 8 XCDs (blockIdx % 8);
  // the parts of one row are given consecutive slots on the same XCD so the
  // second part finds the row's K/V blocks in that XCD's L2.
  const int nrows = p.B * p.Hkv * p.Qb;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int chunk = slot / p.parts;
  const int part = slot - chunk * p.parts;
  const int roww = chunk * 8 + xcd;
  if (roww >= nrows) return;  // uniform: before any barrier
  int b, g, qb;
  if (MODE == kModeCsr && p.row_order != nullptr) {
    const int r = __builtin_amdgcn_readfirstlane(p.row_order[roww]);
    if (r < 0 || r >= nrows) return;  // uniform: before any barrier
    qb = r % p.Qb;
    const int bg = r / p.Qb;
    g = bg % p.Hkv;
    b = bg / p.Hkv;
  } else {
    // Heaviest (last) query blocks first: causal rows grow with qb.  KV head
    // varies fastest, so XCD x always serves KV head x % Hkv (Hkv | 8).
    const int bh = p.B * p.Hkv;
    qb = p.Qb - 1 - roww / bh;
    const int bg = roww - (roww / bh) * bh;
    b = bg / p.Hkv;
    g = bg - b * p.Hkv;
  }
  // In 8-wave workgroups whose parts split the 2G tiles evenly, tiles are
  // half-major (t = half * G + head): the waves of a part share their query
  // rows, and the capture form needs every query head of a half in one part
  // for the group average (dense causal at cfg2: 7.07-7.13 -> 6.93-6.95 ms).
  // Otherwise tile t is query head t / 2, half t % 2 (one head per part in
  // the 2-wave single-head shape), and the spare waves of the last part are
  // inactive.  The per-query-head mask walker derives the heads of a part
  // from the same order.
  const bool half_major = CAP || (WAVES == 8 && p.tpp * p.parts == 2 * p.G);
  bool active;
  int hq, qhalf;
  if (half_major) {
    const int t = part * p.tpp + wave;
    active = wave < p.tpp;
    qhalf = active ? t / p.G : 0;
    hq = active ? t - qhalf * p.G : 0;
  } else {
    const int tile = part * p.tpp + wave;
    active = wave < p.tpp && tile < 2 * p.G;
    hq = active ? (tile >> 1) : 0;
    qhalf = tile & 1;
  }
  const int head = g * p.G + hq;
  const int q0 = qb * kBlock + qhalf * 32;  // first query of this wave's tile
  const int qin = qhalf * 32 + l32;         // this lane's query row in the block

  // ---- Q fragment (B operand of S^T = K Q^T), resident for the whole row
  uint4 qf[KS];
  raw8_t<TIn> qraw[KS];
  {
    const int64_t qrs = p.qs[2] * EB;
    int nq = p.T - q0;
    nq = nq < 0 ? 0 : (nq > 32 ? 32 : nq);
    if (!active) nq = 0;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        static_cast<const char*>(p.q) + ((int64_t)b * p.qs[0] + (int64_t)head * p.qs[1] + (int64_t)q0 * p.qs[2]) * EB,
        (uint32_t)(nq * qrs));
    const int vq = l32 * (int)qrs + 8 * hl * EB;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qraw[kk] = buf_load8<TIn>(rq, vq + 16 * kk * EB);
  }
  // The fragments are converted (prescaled, or rounded from fp32) only once
  // the first key block's loads are in flight, so the Q and K/V round trips
  // overlap instead of running back to back.
  bool q_ready = false;
  auto convert_q = [&]() {
    q_ready = true;
    if (p.prescale) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) qf[kk] = to_mfma_scaled<TIn, F16>(qraw[kk], p.qmul, true);
    } else {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) qf[kk] = raw_to_mfma<TIn, F16>(qraw[kk]);
    }
  };
  // The summary form converts at once: its registers are tighter.
  if constexpr (SUMM) convert_q();

  // ---- per-lane staging offsets, constant across blocks
  const char* kbase = static_cast<const char*>(p.k) + ((int64_t)b * p.ks[0] + (int64_t)g * p.ks[1]) * EB;
  const char* vbase = static_cast<const char*>(p.v) + ((int64_t)b * p.vs[0] + (int64_t)g * p.vs[1]) * EB;
  const int krs = (int)(p.ks[2] * EB), vrs = (int)(p.vs[2] * EB);
  int koff[KCH], klds[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = tid + i * NTHR;
    const int key = c / KROWCH, dc = c % KROWCH;
    koff[i] = c < KCHUNKS ? key * krs + dc * 8 * EB : kOutOfRange;
    klds[i] = key * KSTR + dc * 8;
  }
  int voff[KCH], vlds[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = tid + i * NTHR;
    const int key = c / KROWCH, dc = c % KROWCH;
    voff[i] = c < KCHUNKS ? key * vrs + dc * 8 * EB : kOutOfRange;
    vlds[i] = key * VSTR + dc * 8;
  }

  raw8_t<TIn> kst[KCH];
  raw8_t<TIn> vst[KCH];

  auto load_block = [&](int blk) {
    const int t0 = blk * kBlock;
    int nk = p.T - t0;
    nk = nk > kBlock ? kBlock : nk;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)t0 * krs, (uint32_t)(nk * krs));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + (int64_t)t0 * vrs, (uint32_t)(nk * vrs));
#pragma unroll
    for (int i = 0; i < KCH; ++i) kst[i] = buf_load8<TIn>(rk, koff[i]);
#pragma unroll
    for (int i = 0; i < KCH; ++i) vst[i] = buf_load8<TIn>(rv, voff[i]);
  };

  auto store_block = [&](int buf) {
    uint16_t* Ks = smem + buf * BUF;
    uint16_t* Vs = Ks + KTILE;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      if ((KCHUNKS % NTHR) == 0 || tid + i * NTHR < KCHUNKS) {
        *reinterpret_cast<uint4*>(Ks + klds[i]) = raw_to_mfma<TIn, F16>(kst[i]);
        *reinterpret_cast<uint4*>(Vs + vlds[i]) = raw_to_mfma<TIn, F16>(vst[i]);
      }
    }
  };

  // Producer form: the last wave (which owns no tile) stages every K/V block
  // alone, so the tile waves carry no staging registers or copy work.  It
  // stages by loads straight into LDS (buffer_load ... lds: lane l of an
  // instruction writes LDS bytes [16 l, 16 l + 16) after the M0 base): the
  // tiles' padded rows are covered granule by granule, each lane fetching
  // the 16 K/V bytes that belong at its granule, and the pad granules read
  // out of range (zeros, no memory traffic).  The barrier after a block
  // waits for these loads (vmcnt), as it waited for the register copies.
  constexpr int PKCH = KCHUNKS / 64;  // K chunks per lane of one wave (summary chunks)
  static_assert(KCHUNKS % 64 == 0, "producer lanes split the block evenly");
  constexpr int KG = KSTR / 8, VG = VSTR / 8;  // 16-byte granules per LDS row, data and pad
  static_assert(KSTR % 8 == 0 && VSTR % 8 == 0, "tile rows are whole 16-byte granules");
  auto dma_off = [&](int i, int G, int rs) {
    const int gidx = 64 * i + lane, row = gidx / G, col = gidx - row * G;
    return col < KROWCH ? row * rs + col * 16 : kOutOfRange;
  };
  int kdma[PROD ? KG : 1], vdma[PROD ? VG : 1];  // this lane's offsets, the same for every block
  if constexpr (PROD) {
#pragma unroll
    for (int i = 0; i < KG; ++i) kdma[i] = dma_off(i, KG, krs);
#pragma unroll
    for (int i = 0; i < VG; ++i) vdma[i] = dma_off(i, VG, vrs);
  }
  auto produce = [&](int blk, int buf) {
    if constexpr (EB == 2) {
      const int t0 = blk * kBlock;
      int nk = p.T - t0;
      nk = nk > kBlock ? kBlock : nk;
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)t0 * krs, (uint32_t)(nk * krs));
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + (int64_t)t0 * vrs, (uint32_t)(nk * vrs));
      uint16_t* Ks = smem + buf * BUF;
#pragma unroll
      for (int i = 0; i < KG; ++i)
        buffer_load_lds16(rk, Ks + 512 * i, kdma[i]);
#pragma unroll
      for (int i = 0; i < VG; ++i)
        buffer_load_lds16(rv, Ks + KTILE + 512 * i, vdma[i]);
    }
  };

  float m_use = -INFINITY;  // softmax reference point (scaled, log2 domain)
  float l_run = 0.f;        // running sum over this lane half's keys
  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16_t{};

  // The block step in three pieces: S^T = K Q^T into (sc0, sc1); the online
  // softmax of those scores into the packed P fragments pk (and the O and
  // l rescale); O^T += V^T P^T.
  f32x16_t sc0, sc1;
  uint4 pk[2][2];
  // LDS fragment reads are interleaved with the MFMAs that consume them,
  // kLookahead k-steps ahead, so the waves' LDS traffic overlaps their
  // matrix-core work instead of running as a separate phase in which all
  // waves of the workgroup contend for LDS.  The order is pinned by
  // scheduling barriers in the S^T loop and scheduling-group barriers in the
  // P.V loop; without the former the scheduler reused one register quad for
  // every K fragment, one read in flight per MFMA.
  auto scores = [&](const uint16_t* Ks) {
    const uint16_t* kp = Ks + l32 * KSTR + 8 * hl;
    uint4 a0[KS], a1[KS];
    auto rd = [&](int kk) {
      a0[kk] = *reinterpret_cast<const uint4*>(kp + 16 * kk);
      a1[kk] = *reinterpret_cast<const uint4*>(kp + 32 * KSTR + 16 * kk);
    };
#pragma unroll
    for (int kk = 0; kk < kLookahead; ++kk) rd(kk);
    f32x16_t s0 = f32x16_t{}, s1 = f32x16_t{};
    // Scheduling barriers pin the order: the reads of step kk + kLookahead
    // are issued before the MFMAs of step kk, so the fragments of three steps
    // are live in distinct registers and each MFMA waits only for its own.
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (kk + kLookahead < KS) rd(kk + kLookahead);
      __builtin_amdgcn_sched_barrier(0);
      s0 = mfma32x32x16<F16>(a0[kk], qf[kk], s0);
      s1 = mfma32x32x16<F16>(a1[kk], qf[kk], s1);
      __builtin_amdgcn_sched_barrier(0);
    }
    sc0 = s0;
    sc1 = s1;
  };
  // General attention mask: the 32 values this lane adds to its scores of a
  // key block (register r of key tile c holds key 32c + 8(r/4) + 4(lane/32)
  // + r%4 of query q0 + l32), loaded before the block's S^T MFMAs.
  // The raw mask bits of the next block are fetched while the current one
  // finishes (after its softmax), so their latency hides behind its P.V,
  // the barrier and the next block's S^T MFMAs.
  //  * Row pieces (amask_rows16, and the block's 64 keys inside the mask):
  //    the wave's 32 query rows are read as 16-byte pieces along each row
  //    (64 * eb bytes per row, so 2, 4 or 8 loads for 1, 2 or 4-byte
  //    elements, each touching 64 * 16 / (64 * eb) rows' lines), then
  //    turned into the score layout through a wave-private LDS region.
  //    Reading each lane's 4-key groups directly instead touches 32 rows'
  //    lines per load, 8 loads per block, and the address units bound it.
  //  * Otherwise group 4c + j of amr holds keys 32c + 8j + 4(lane/32) .. + 3
  //    of query q0 + l32, read directly.
  uint4 amr[AMASK ? 8 : 1];
  bool am_rows = false;  // wave-uniform: amr holds row pieces
  constexpr int kAmRowWords = 68;  // LDS row of the staging region: 256 + 16 bytes
  __shared__ __attribute__((aligned(16))) uint32_t amlds[AMASK ? WAVES * 32 * kAmRowWords : 1];
  auto fetch_amask = [&](int blk) {
    if constexpr (AMASK) {
#pragma unroll
      for (int g8 = 0; g8 < 8; ++g8) amr[g8] = uint4{0u, 0u, 0u, 0u};
      am_rows = false;
      if (blk < 0) return;
      const int mh = p.amask_heads > 1 ? head : 0;
      const int64_t rbase = (int64_t)b * p.ams[0] + (int64_t)mh * p.ams[1];
      const int eb = p.amask_dtype == SPRUCE_DTYPE_F32 ? 4 : (p.amask_dtype == SPRUCE_DTYPE_U8 ? 1 : 2);
      if (p.amask_rows16 && blk * kBlock + kBlock <= p.amask_tk) {
        am_rows = true;
        const int lpr = 4 * eb;          // lanes per row (16 bytes each)
        const int rpi = 64 / lpr;        // rows per load
        const int rr = lane / lpr, cb = (lane % lpr) * 16;
        const char* mbase = static_cast<const char*>(p.amask);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = i * rpi + rr;
          if (i < 32 / rpi && q0 + r < p.T)
            amr[i] = *reinterpret_cast<const uint4*>(
                mbase + (rbase + (int64_t)(q0 + r) * p.ams[2] + (int64_t)blk * kBlock) * eb + cb);
        }
        return;
      }
      const int qt = q0 + l32;
      if (qt < p.T) {
        const int64_t row = rbase + (int64_t)qt * p.ams[2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key0 = blk * kBlock + 32 * c + 8 * j + 4 * hl;
            amr[4 * c + j] = amask_fetch4(p, row + key0, p.T - key0);
          }
      }
    }
  };
  // Row pieces -> this lane's 4-key groups, through the wave's LDS rows.
  auto stage_amask = [&]() {
    if constexpr (AMASK) {
      if (!am_rows) return;
      const int eb = p.amask_dtype == SPRUCE_DTYPE_F32 ? 4 : (p.amask_dtype == SPRUCE_DTYPE_U8 ? 1 : 2);
      const int lpr = 4 * eb, rpi = 64 / lpr;
      const int rr = lane / lpr, cb = (lane % lpr) * 16;
      char* reg = reinterpret_cast<char*>(amlds + wave * 32 * kAmRowWords);
      constexpr int RB = kAmRowWords * 4;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < 32 / rpi) *reinterpret_cast<uint4*>(reg + (i * rpi + rr) * RB + cb) = amr[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const char* mine = reg + l32 * RB + 4 * hl * eb;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const char* src = mine + (32 * c + 8 * j) * eb;
          if (eb == 4) {
            amr[4 * c + j] = *reinterpret_cast<const uint4*>(src);
          } else if (eb == 2) {
            const uint2 x = *reinterpret_cast<const uint2*>(src);
            amr[4 * c + j] = uint4{x.x, x.y, 0u, 0u};
          } else {
            amr[4 * c + j] = uint4{*reinterpret_cast<const uint32_t*>(src), 0u, 0u, 0u};
          }
        }
      // The next block's stores into these rows come after these reads in
      // the wave's own order.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  };
  // sb: per-key score bias of a summary chunk (null for a key block).
  // vb: validity bits of the block's 64 keys (key padding; all set otherwise).
  auto softmax = [&](bool diag, const float* sb, uint64_t vb) {
    f32x16_t s0 = sc0, s1 = sc1;
    if constexpr (AMASK) {
      stage_amask();
      // Added in raw score units: (s + mask * log2(e) / cs) * cs.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v0[4], v1[4];
        amask_unpack4(p.amask_dtype, amr[j], v0);
        amask_unpack4(p.amask_dtype, amr[4 + j], v1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          s0[4 * j + t] += v0[t] * p.amask_mul;
          s1[4 * j + t] += v1[t] * p.amask_mul;
        }
      }
    }
    if constexpr (KVAL) {
      // Register r of key tile c holds key 32c + 8(r/4) + 4(lane/32) + r%4.
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + 4 * hl + (r & 3);
        if (!((vb >> kr) & 1ull)) s0[r] = -INFINITY;
        if (!((vb >> (32 + kr)) & 1ull)) s1[r] = -INFINITY;
      }
    }
    if (diag) {
      // Register r of key tile c holds key 32c + 8(r/4) + 4(lane/32) + r%4.
      const int thr = qin - 4 * hl;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + (r & 3);
        if (kr > thr) s0[r] = -INFINITY;
        if (32 + kr > thr) s1[r] = -INFINITY;
      }
    }
    if (sb != nullptr) {
      // Summary keys: add log(count) in raw score units; no causal mask
      // (sparse/attention.py:252-258).  Register 4j+t of key tile c holds
      // key 32c + 8j + 4(lane/32) + t.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 b0 = *reinterpret_cast<const float4*>(sb + 8 * j + 4 * hl);
        const float4 b1 = *reinterpret_cast<const float4*>(sb + 32 + 8 * j + 4 * hl);
        s0[4 * j] += b0.x; s0[4 * j + 1] += b0.y; s0[4 * j + 2] += b0.z; s0[4 * j + 3] += b0.w;
        s1[4 * j] += b1.x; s1[4 * j + 1] += b1.y; s1[4 * j + 2] += b1.z; s1[4 * j + 3] += b1.w;
      }
    }
    float mx = fmaxf(s0[0], s0[1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s0[r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[r]);
    mx = half_max(mx);
    const float cand = mx * p.cs;
    if (__ballot(cand > m_use + kRescaleThreshold) != 0) {
      const float m_new = fmaxf(m_use, cand);
      // With key padding a padded query row can still have no usable key
      // while others in the wave do: keep its (empty) state as it is.
      const float alpha = ((KVAL || AMASK) && m_new == -INFINITY) ? 1.f : fast_exp2(m_use - m_new);
      m_use = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    }
    // A lane whose keys so far are all -inf (a summary-only row) keeps
    // m_use = -inf; exp2(-inf) = 0 needs a finite offset there.
    const float nm = ((KVAL || AMASK || sb != nullptr) && m_use == -INFINITY) ? 0.f : -m_use;
    float psum = 0.f;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      uint32_t w0[4], w1[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = fast_exp2(fmaf(s0[8 * h2 + 2 * e], p.cs, nm));
        const float x1 = fast_exp2(fmaf(s0[8 * h2 + 2 * e + 1], p.cs, nm));
        const float y0 = fast_exp2(fmaf(s1[8 * h2 + 2 * e], p.cs, nm));
        const float y1 = fast_exp2(fmaf(s1[8 * h2 + 2 * e + 1], p.cs, nm));
        psum += (x0 + x1) + (y0 + y1);
        w0[e] = pack2<F16>(x0, x1);
        w1[e] = pack2<F16>(y0, y1);
      }
      pk[0][h2] = uint4{w0[0], w0[1], w0[2], w0[3]};
      pk[1][h2] = uint4{w1[0], w1[1], w1[2], w1[3]};
    }
    l_run += psum;
  };
  // O^T += V^T P^T, V^T fragments interleaved like the K fragments;
  // consecutive MFMAs go to different output tiles (dt fastest), so no MFMA
  // waits on the previous one's result.  The P^T fragment pk[c][h2] holds
  // keys K0 + 4 hl + 0..3 and K0 + 8 + 4 hl + 0..3 (K0 = 32 c + 16 h2: the
  // S^T accumulator order) for query column l32; the matching V^T fragment
  // of d = 32 dt + l32 is two transposing reads of 4 keys each.  Source lane
  // s of 16-lane group gr points at keys K0 + 4 (gr / 2) + s / 4 (+ 8),
  // dims 32 dt + 16 (gr % 2) + 4 (s % 4) + 0..3.
  const int vlane = (4 * hl + ((lane & 15) >> 2)) * VSTR + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  auto pv = [&](const uint16_t* Vs) {
    const uint16_t* vp = Vs + vlane;
    uint4 va[DT * 4];
#pragma unroll
    for (int i = 0; i < DT * 4; ++i) {
      const int dt = i % DT, ch = i / DT, c = ch >> 1, h2 = ch & 1;
      const uint16_t* a = vp + (32 * c + 16 * h2) * VSTR + 32 * dt;
      const uint2 lo = lds_read_tr16(a), hi = lds_read_tr16(a + 8 * VSTR);
      va[i] = uint4{lo.x, lo.y, hi.x, hi.y};
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4 * kLookahead, 0);
#pragma unroll
    for (int i = 0; i < DT * 4 - 2 * kLookahead; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * kLookahead, 0);
#pragma unroll
    for (int i = 0; i < DT * 4; ++i) {
      const int dt = i % DT, ch = i / DT, c = ch >> 1, h2 = ch & 1;
      acc[dt] = mfma32x32x16<F16>(va[i], pk[c][h2], acc[dt]);
    }
  };
  // next_blk: the block after this one (-1: none), whose mask bits are
  // fetched once this block's scores hold its own (AMASK only).
  auto compute = [&](int buf, bool diag, const float* sb, uint64_t vb, int next_blk) {
    const uint16_t* Ks = smem + buf * BUF;
    scores(Ks);
    softmax(diag, sb, vb);
    fetch_amask(next_blk);
    pv(Ks + KTILE);
  };
  // Key padding: this lane's validity byte of block `blk` (loaded one block
  // ahead; the ballot over the wave gives the block's 64 bits).
  auto vbyte = [&](int blk) -> uint32_t {
    if constexpr (KVAL) {
      const int key = blk * kBlock + lane;
      return key < p.T ? (uint32_t)p.kvalid[(int64_t)b * p.kvs + key] : 0u;
    } else {
      return 1u;
    }
  };
  auto vbits = [&](uint32_t raw) -> uint64_t { return KVAL ? __ballot(raw != 0u) : ~0ull; };

  // ---- residual summaries of the row (SUMM): entry e is prototype e % P
  // of the row's (e / P)-th node, appended after the exact keys as chunks of
  // 64 keys (sparse/attention.py:232-265).  Missing nodes and empty
  // prototypes get a -inf bias, so they add exactly zero weight.
  __shared__ __attribute__((aligned(16))) float sbias[SUMM ? 2 : 1][kBlock];
  const int32_t* nrow =
      SUMM ? p.snode + (int64_t)b * p.sns[0] + (int64_t)g * p.sns[1] + (int64_t)qb * p.sns[2] : nullptr;
  // The row's summary entries: listed nodes (up to the last valid one) x P.
  auto summary_entries = [&]() __attribute__((always_inline)) {
    int nn = 0;  // one past the last listed node (uniform)
    for (int j0 = 0; j0 < p.S; j0 += 64) {
      const int j = j0 + lane;
      const int v = j < p.S ? nrow[(int64_t)j * p.sns[3]] : -1;
      const uint64_t m = __ballot(v >= 0 && v < p.N);
      if (m) nn = j0 + 64 - __builtin_clzll(m);
    }
    return nn * p.P;
  };
  const int64_t bg = (int64_t)b * p.Hkv + g;
  auto node_of = [&](int en, int E) __attribute__((always_inline)) {
    if (en >= E) return -1;
    const int v = nrow[(int64_t)(en / p.P) * p.sns[3]];
    return (v >= 0 && v < p.N) ? v : -1;
  };
  // Table row offset (elements) of entry en of node `node`, dims d0..
  auto row_at = [&](int en, int node, int d0) __attribute__((always_inline)) { return ((bg * p.N + node) * p.P + en % p.P) * (int64_t)D + d0; };
  auto load_row8 = [&](const void* base, int en, int node, int d0) __attribute__((always_inline)) {
    if (node < 0) return uint4{0u, 0u, 0u, 0u};
    if (EB == 2 && p.sum16)  // a copy in the input type (never for float32 inputs)
      return *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + row_at(en, node, d0));
    const float4* s = reinterpret_cast<const float4*>(static_cast<const float*>(base) + row_at(en, node, d0));
    const float4 x = s[0], y = s[1];
    return uint4{pack2<F16>(x.x, x.y), pack2<F16>(x.z, x.w), pack2<F16>(y.x, y.y), pack2<F16>(y.z, y.w)};
  };
  // Producer form: the producer wave stages each chunk while the tile waves
  // compute the previous one (the first chunk while they compute the row's
  // last key block), with the key blocks' barrier sequence.  Lane l holds
  // the node of entry e0 + l; the 16-byte pieces of the 64 table rows are
  // spread over the lanes as in the key blocks' staging, each taking its
  // entry's node from the owning lane.  A 16-bit copy of the table is staged
  // with all of a chunk's loads in flight at once (the producer returns
  // after the output barrier, so none of the tile waves' registers are live
  // here); a float32 table in batches of kSumBatch pieces per lane (2
  // float4 loads each), rounded on the way.
  constexpr int kSumBatch = PKCH / 2;
  auto stage_rows = [&](const void* table, uint16_t* dst, int stride, int e0, int mine) __attribute__((always_inline)) {
#pragma unroll
    for (int i0 = 0; i0 < PKCH; i0 += kSumBatch) {
      float4 x[2 * kSumBatch];
#pragma unroll
      for (int i = 0; i < kSumBatch; ++i) {
        const int c = lane + 64 * (i0 + i), key = c / KROWCH, dc = c % KROWCH;
        const int node = __shfl(mine, key);
        if (node >= 0) {
          const float4* src =
              reinterpret_cast<const float4*>(static_cast<const float*>(table) + row_at(e0 + key, node, dc * 8));
          x[2 * i] = src[0];
          x[2 * i + 1] = src[1];
        } else {
          x[2 * i] = x[2 * i + 1] = float4{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int i = 0; i < kSumBatch; ++i) {
        const int c = lane + 64 * (i0 + i), key = c / KROWCH, dc = c % KROWCH;
        const float4 u = x[2 * i], w = x[2 * i + 1];
        *reinterpret_cast<uint4*>(dst + key * stride + dc * 8) =
            uint4{pack2<F16>(u.x, u.y), pack2<F16>(u.z, u.w), pack2<F16>(w.x, w.y), pack2<F16>(w.z, w.w)};
      }
    }
  };
  BlockIter<MODE> it;
  it.init(p, b, g, qb, part, hq, lane, half_major);
  int cur_id = 0;
  bool cur_en = false;
  int buf = 0;
  const bool any_block = it.next(cur_id, cur_en);
  if constexpr (PROD) {
    // Same barrier sequence on both sides: one before the first block and
    // one between consecutive blocks.
    if (wave == WAVES - 1) {
      if (any_block) {
        produce(cur_id, 0);
        __syncthreads();
        while (true) {
          int nid = 0;
          bool nen = false;
          if (!it.next(nid, nen)) break;
          produce(nid, buf ^ 1);
          __syncthreads();
          buf ^= 1;
        }
      }
      if constexpr (SUMM) {
        const int E = summary_entries();
        int mine = node_of(lane, E);  // lane l: the node of entry e0 + l
        for (int e0 = 0; e0 < E; e0 += kBlock) {
          buf ^= 1;  // its last readers finished before the previous barrier
          uint16_t* Ks = smem + buf * BUF;
          const int next = node_of(e0 + kBlock + lane, E);  // the next chunk's, read ahead
          sbias[buf][lane] =
              mine < 0 ? -INFINITY : p.slog[((int64_t)b * p.N + mine) * p.P + (e0 + lane) % p.P] * p.sbias;
          if (p.sum16) {
            uint4 xk[PKCH], xv[PKCH];
#pragma unroll
            for (int i = 0; i < PKCH; ++i) {
              const int c = lane + 64 * i, key = c / KROWCH, dc = c % KROWCH;
              const int node = __shfl(mine, key);
              const int64_t off = node >= 0 ? row_at(e0 + key, node, dc * 8) : 0;
              xk[i] = node >= 0 ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.skey) + off)
                                : uint4{0u, 0u, 0u, 0u};
              xv[i] = node >= 0 ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.sval) + off)
                                : uint4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int i = 0; i < PKCH; ++i) {
              const int c = lane + 64 * i, key = c / KROWCH, dc = c % KROWCH;
              *reinterpret_cast<uint4*>(Ks + key * KSTR + dc * 8) = xk[i];
              *reinterpret_cast<uint4*>(Ks + KTILE + key * VSTR + dc * 8) = xv[i];
            }
          } else {
            stage_rows(p.skey, Ks, KSTR, e0, mine);
            stage_rows(p.sval, Ks + KTILE, VSTR, e0, mine);
          }
          __syncthreads();
          mine = next;
        }
        __syncthreads();  // the output staging's barrier below
        return;
      }
    } else if (any_block) {
      if (!q_ready) convert_q();
      uint32_t vcur = vbyte(cur_id);
      fetch_amask(cur_id);
      __syncthreads();
      while (true) {
        int nid = 0;
        bool nen = false;
        const bool more = it.next(nid, nen);
        const uint32_t vnext = more ? vbyte(nid) : 0u;
        if (active && cur_en) compute(buf, cur_id == qb, nullptr, vbits(vcur), more ? nid : -1);
        if (!more) break;
        __syncthreads();
        buf ^= 1;
        cur_id = nid;
        cur_en = nen;
        vcur = vnext;
      }
    }
  } else if (any_block) {
    uint32_t vcur = vbyte(cur_id);
    load_block(cur_id);
    fetch_amask(cur_id);
    if (!q_ready) convert_q();
    store_block(0);
    __syncthreads();
    while (true) {
      int nid = 0;
      bool nen = false;
      const bool more = it.next(nid, nen);
      const uint32_t vnext = more ? vbyte(nid) : 0u;
      if (more) load_block(nid);
      if (active && cur_en) compute(buf, cur_id == qb, nullptr, vbits(vcur), more ? nid : -1);
      if (!more) break;
      store_block(buf ^ 1);
      __syncthreads();
      buf ^= 1;
      cur_id = nid;
      cur_en = nen;
      vcur = vnext;
    }
  }

  if constexpr (SUMM) {
    const int E = summary_entries();
    if (E > 0 && !q_ready) convert_q();  // the row listed no exact block
    if constexpr (PROD) {
      // The tile waves' side of produce_summaries (the producer returned).
      for (int e0 = 0; e0 < E; e0 += kBlock) {
        buf ^= 1;
        __syncthreads();
        if (active) compute(buf, false, sbias[buf], ~0ull, -1);
      }
    } else {
      for (int e0 = 0; e0 < E; e0 += kBlock) {
        buf ^= 1;  // its last reader finished before the previous barrier
        uint16_t* Ks = smem + buf * BUF;
        uint16_t* Vs = Ks + KTILE;
        for (int c = tid; c < KCHUNKS; c += NTHR) {
          const int key = c / KROWCH, dc = c % KROWCH;
          const int en = e0 + key;
          *reinterpret_cast<uint4*>(Ks + key * KSTR + dc * 8) = load_row8(p.skey, en, node_of(en, E), dc * 8);
        }
        for (int c = tid; c < KCHUNKS; c += NTHR) {
          const int key = c / KROWCH, dc = c % KROWCH;
          const int en = e0 + key;
          *reinterpret_cast<uint4*>(Vs + key * VSTR + dc * 8) = load_row8(p.sval, en, node_of(en, E), dc * 8);
        }
        if (tid < kBlock) {
          const int en = e0 + tid;
          const int node = node_of(en, E);
          sbias[buf][tid] = node < 0 ? -INFINITY : p.slog[((int64_t)b * p.N + node) * p.P + en % p.P] * p.sbias;
        }
        __syncthreads();
        if (active) compute(buf, false, sbias[buf], ~0ull, -1);
      }
    }
  }

  if constexpr (CAP) {
    // Every block 0..qb was walked in order, so buffer `buf` still holds the
    // diagonal K tile and the other buffer has no readers left.
    constexpr int QRS = D + 8;
    static_assert(WAVES * 32 * QRS <= 2 * BUF, "query staging must fit the K/V tiles");
    const int64_t bg = (int64_t)b * p.Hkv + g;
    if (part == 0) {
      int n = p.T - qb * kBlock;
      n = n > kBlock ? kBlock : n;
      capture_key_prototypes<D, KSTR, NTHR, F16>(smem + buf * BUF, reinterpret_cast<float*>(smem + (buf ^ 1) * BUF),
                                                 n, p.P,
                                                 static_cast<uint16_t*>(p.kproto) + (bg * p.Qb + qb) * p.P * D, tid);
    }
    __syncthreads();
    if (active) {
      // The Q fragments are the raw model-dtype rows (never prescaled here).
      uint16_t* qd = smem + (wave * 32 + l32) * QRS + 8 * hl;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) *reinterpret_cast<uint4*>(qd + 16 * kk) = qf[kk];
    }
    __syncthreads();
    const int nh = p.tpp / p.G;
    const int t_first = qb * kBlock + part * nh * 32;
    capture_group_average<D, NTHR, F16>(smem, QRS, p.G, nh, p.inv_rep, t_first, p.T,
                                        static_cast<uint16_t*>(p.qgrp) + (bg * p.T + t_first) * D, tid);
  }

  if constexpr (EB == 2) {
    // The output tile goes through LDS so that every store writes whole
    // 16-byte pieces of 256-byte rows (the accumulator layout would write 8
    // bytes to each of 64 rows per instruction).  The K/V tiles are free
    // once every wave is past its last block.
    constexpr int OSTR = D + 8;
    static_assert(WAVES * 32 * OSTR <= 2 * BUF, "output staging must fit the K/V tiles");
    __syncthreads();
    if (!active) return;
    const float lt = half_sum(l_run);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* ot = smem + wave * 32 * OSTR;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = dt * 32 + 8 * j + 4 * hl;
        const uint32_t w0 = pack2<F16>(acc[dt][4 * j] * inv, acc[dt][4 * j + 1] * inv);
        const uint32_t w1 = pack2<F16>(acc[dt][4 * j + 2] * inv, acc[dt][4 * j + 3] * inv);
        *reinterpret_cast<uint2*>(ot + l32 * OSTR + d) = uint2{w0, w1};
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t ors = p.os[2] * EB;
    int nq = p.T - q0;
    nq = nq < 0 ? 0 : (nq > 32 ? 32 : nq);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(
        static_cast<char*>(p.o) + ((int64_t)b * p.os[0] + (int64_t)head * p.os[1] + (int64_t)q0 * p.os[2]) * EB,
        (uint32_t)(nq * ors));
    constexpr int CH = D / 8;  // 16-byte pieces per row
#pragma unroll
    for (int i = 0; i < 32 * CH / 64; ++i) {
      const int c = i * 64 + lane;
      const int row = c / CH, ch = c % CH;
      const uint4 v = *reinterpret_cast<const uint4*>(ot + row * OSTR + ch * 8);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v),
                                             ro, row * (int)ors + ch * 16, 0, 0);
    }
    return;
  }
  if (!active) return;
  const float lt = half_sum(l_run);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const int64_t ors = p.os[2] * EB;
  int nq = p.T - q0;
  nq = nq < 0 ? 0 : (nq > 32 ? 32 : nq);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(
      static_cast<char*>(p.o) + ((int64_t)b * p.os[0] + (int64_t)head * p.os[1] + (int64_t)q0 * p.os[2]) * EB,
      (uint32_t)(nq * ors));
  const int vo = l32 * (int)ors;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = dt * 32 + 8 * j + 4 * hl;
      const float o0 = acc[dt][4 * j] * inv, o1 = acc[dt][4 * j + 1] * inv;
      const float o2 = acc[dt][4 * j + 2] * inv, o3 = acc[dt][4 * j + 3] * inv;
      if constexpr (EB == 2) {
        const uint32_t w[2] = {pack2<F16>(o0, o1), pack2<F16>(o2, o3)};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, w),
                                              ro, vo + d * EB, 0, 0);
      } else {
        const float f[4] = {o0, o1, o2, o3};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, f),
                                               ro, vo + d * EB, 0, 0);
      }
    }
}

// ------------------------------------------------------------------ launch
constexpr bool kUseProducer = true;

struct LaunchShape {
  int waves;
  int parts;
  int tpp;  // tiles per part (<= waves)
};

// Tiles of one (batch, KV head, query block) row: 2 per query head.  Rows of
// 5 or more tiles per part use 8-wave workgroups split into as few parts as
// possible, spare waves helping only to stage K/V: every extra part fetches
// the row's K/V blocks again, and at two waves per SIMD a CU holds one such
// workgroup either way.  Measured at T = 32K, 10% density: G = 7 (14 tiles,
// 7 per part) 3% faster than 7-wave workgroups; G = 3, 5, 6 25-50% faster
// than the 2- and 4-wave splits.  Smaller rows keep one wave per tile.
inline LaunchShape choose_shape(int variant, int G) {
  const int tiles = 2 * G;
  if (variant == SPRUCE_VARIANT_SINGLE_HEAD_QTILE) return {2, G, 2};
  if (tiles % 8 == 0) return {8, tiles / 8, 8};
  const int parts = (tiles + 7) / 8, tpp = (tiles + parts - 1) / parts;
  if (tpp >= 5) return {8, parts, tpp};
  return tiles % 4 == 0 ? LaunchShape{4, tiles / 4, 4} : LaunchShape{2, tiles / 2, 2};
}

// Block-sparse launches with fewer workgroups than the part has CUs (short
// sequences, few KV heads: 128 rows of one 8-wave part at the reference's
// T = 4096, 8/2-head case) leave CUs idle for the whole launch; there the
// rows are split into 4- or 2-wave parts (one wave per tile) until every CU
// has one, since a second fetch of a row's K/V blocks costs less than an
// idle CU.  Every shape computes the same attention.
constexpr int64_t kComputeUnits = 256;  // MI355X
inline void split_small_grid(AttnParams& p, LaunchShape& s, int variant) {
  if (variant == SPRUCE_VARIANT_SINGLE_HEAD_QTILE) return;
  const int64_t rows = (int64_t)p.B * p.Hkv * p.Qb;
  const int tiles = 2 * p.G;
  while (rows * s.parts < kComputeUnits && s.waves > 2) {
    if (s.waves == 8 && tiles % 4 == 0)
      s = LaunchShape{4, tiles / 4, 4};
    else
      s = LaunchShape{2, tiles / 2, 2};
  }
  p.parts = s.parts;
  p.tpp = s.tpp;
}

template <int D, int WAVES, typename TIn, bool F16, int MODE, bool SUMM, bool CAP = false, bool PROD = false,
          bool KVAL = false, bool AMASK = false>
int launch_attention_t(const AttnParams& p, hipStream_t stream) {
  // Rows are padded to a multiple of the 8 XCDs; the extra workgroups exit.
  const int64_t rows8 = ((int64_t)p.B * p.Hkv * p.Qb + 7) / 8 * 8;
  const int64_t grid = rows8 * p.parts;
  hipLaunchKernelGGL((sparse_prefill_kernel<D, WAVES, TIn, F16, MODE, SUMM, CAP, PROD, KVAL, AMASK>),
                     dim3((unsigned)grid), dim3(WAVES * 64), 0, stream, p);
  return check_launch("sparse_prefill_kernel");
}

template <int MODE, bool SUMM, int D, typename TIn, bool F16, bool KVAL, bool AMASK = false>
int launch_attention_w(const AttnParams& p, int waves, hipStream_t stream) {
  switch (waves) {
    case 2: return launch_attention_t<D, 2, TIn, F16, MODE, SUMM, false, false, KVAL, AMASK>(p, stream);
    case 4: return launch_attention_t<D, 4, TIn, F16, MODE, SUMM, false, false, KVAL, AMASK>(p, stream);
    case 8:
      // A spare wave becomes the K/V producer (16-bit inputs, key blocks only).
      if constexpr (kUseProducer && TIn::bytes == 2)
        if (p.tpp < 8) return launch_attention_t<D, 8, TIn, F16, MODE, SUMM, false, true, KVAL, AMASK>(p, stream);
      return launch_attention_t<D, 8, TIn, F16, MODE, SUMM, false, false, KVAL, AMASK>(p, stream);
    default: return set_error(SPRUCE_EINVAL, "unsupported wave count %d", waves);
  }
}

template <int MODE, bool SUMM = false, bool KVAL = false, bool AMASK = false>
int launch_attention(const AttnParams& p, int D, int dtype, int waves, hipStream_t stream) {
  if (D == 128) {
    if (dtype == SPRUCE_DTYPE_BF16)
      return launch_attention_w<MODE, SUMM, 128, InBF16, false, KVAL, AMASK>(p, waves, stream);
    if (dtype == SPRUCE_DTYPE_F16) return launch_attention_w<MODE, SUMM, 128, InF16, true, KVAL, AMASK>(p, waves, stream);
    return launch_attention_w<MODE, SUMM, 128, InF32, false, KVAL, AMASK>(p, waves, stream);
  }
  if (dtype == SPRUCE_DTYPE_BF16) return launch_attention_w<MODE, SUMM, 64, InBF16, false, KVAL, AMASK>(p, waves, stream);
  if (dtype == SPRUCE_DTYPE_F16) return launch_attention_w<MODE, SUMM, 64, InF16, true, KVAL, AMASK>(p, waves, stream);
  return launch_attention_w<MODE, SUMM, 64, InF32, false, KVAL, AMASK>(p, waves, stream);
}

// Shared argument checks and parameter setup of the three entry points.
int prepare_attention(AttnParams& p, const void* q, const int64_t qs[4], const void* k,
                      const int64_t ks[4], const void* v, const int64_t vs[4], int64_t B,
                      int64_t Hq, int64_t Hkv, int64_t T, int64_t D, float scale, int dtype,
                      int variant, void* out, const int64_t os[4], LaunchShape& shape);

}  // namespace spruce
