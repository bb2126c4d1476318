// Teacher target extraction on gfx950: dense causal softmax attention reduced
// to per-(head, query block, key block) probability mass, without ever forming
// the [T, T] attention matrix, and the row-normalised top-k block targets.
//
// Semantics follow chunked_pool (teacher/chunked_extract.py:91-131):
//   mass[b, h, I, J] = sum over query rows i of block I and keys j of block J,
//   j <= i, of softmax_j(q_i . k_j * scale) over the row's causal keys,
// with query head h reading KV head h / G (the reference repeats K to H heads,
// teacher/chunked_extract.py:83-88,139), and the target post-processing of
// load_teacher (selector/targets.py:104-121): mean over the G query heads of a
// KV group, causal mask, row normalisation with eps, plus the top-k blocks of
// each target row (selector/loss.py:34-46, selector/recall.py:35).
//
// Scores are accumulated in float32 on the matrix cores from the bf16/f16
// inputs as given (the reference rounds QK^T itself to the model dtype
// before its float32 softmax, teacher/chunked_extract.py:119,126).  Q is not
// prescaled: rounding q * scale * log2(e) to bf16 would add a score error
// that grows with the score's magnitude.
//
// The causal (I, J) tiles are walked GQA-packed like the sparse prefill
// kernel (one workgroup per (batch, KV head, query block, part), one 32-row
// tile of one query head per wave, K blocks staged once per workgroup in LDS).
//
// Per score element the loop issues one FMA (s * cs - m, cs = scale *
// log2(e)), one v_exp_f32 and one add; the row max is taken only in the rare
// blocks whose partial sum exceeds kMassCheckSum, not per block.  On gfx950
// v_exp_f32 issues at half the rate of an FMA and does not overlap other VALU
// work, so per element these three already take about as long as the MFMA
// work of the score; any further VALU work per element shows in the time.
//
// A row's mass needs its final softmax denominator l before its 64 rows are
// summed, so one of two schedules is used:
//   single pass (when its scratch fits, see kSinglePassScratchMax): online
//     row reference point and denominator, and for every J the row's partial
//     sum e_J = sum_j exp2(s_j - m_r), staged in an LDS ring of kRing blocks
//     whose entries all share one reference point m_r (a raise of the row's
//     reference point rescales the ring's earlier entries); a full ring goes
//     to scratch as 4 bytes per row and J plus m_r once per row and ring, and
//     the row's last ring stays in LDS.  Once the row is complete the wave
//     sums e_J * exp2(m_r - m) / l over its 32 rows in a fixed butterfly
//     order.  QK^T runs once.
//   two passes (longer sequences): pass 1 keeps only the row reference point
//     and denominator; pass 2 recomputes the scores and sums exp2(s - m) / l
//     over each 32-row x 64-key tile.  QK^T runs twice.
// Both write one float per (tile half, J) into a [B, H, 2, Qb, Qb] workspace;
// mass = half0 + half1 (exactly two addends, order-independent).
#include <type_traits>

#include "attention_impl.h"

namespace spruce {

struct MassParams {
  const void* q;
  const void* k;
  int64_t qs[4], ks[4];
  int B, Hq, Hkv, T, G, Qb, parts;
  int tpp;      // tiles per part: waves 0..tpp-1 own a tile
  float cs;     // scale * log2(e)
  float* stats;  // [B, Hq, T, 2]: (row max in log2 units, row sum), two-pass only
  float* part;   // [B, Hq, 2, Qb, Qb]
  float* rowe;   // single pass: [B, Hq, 2, Qb(Qb+1)/2, 32] e_J per row (query block I at I(I+1)/2)
  float* rowm;   // single pass: [B, Hq, 2, ring_slots(Qb), 32] m_r per row and ring
};

// Key blocks whose per-row partials a wave stages in LDS before one copy to
// the single-pass scratch; they share one reference point per row.
constexpr int kRing = 16;

// Rings of the query blocks before I: sum over i < I of ceil((i + 1) / kRing).
__host__ __device__ inline int64_t ring_slots(int64_t I) {
  const int64_t q = I / kRing, r = I % kRing;
  return kRing * q * (q + 1) / 2 + r * (q + 1);
}

// Single-pass scratch is B*Hq*(Qb*(Qb+1)*128 + ring_slots(Qb)*256) bytes
// (243 MB at T=16K, 28 heads); above kSinglePassScratchMax the two-pass
// schedule is used instead.
constexpr int64_t kSinglePassScratchMax = (int64_t)4 << 30;

inline int64_t single_pass_e_bytes(int64_t B, int64_t Hq, int64_t Qb) { return B * Hq * Qb * (Qb + 1) * 128; }

inline int64_t single_pass_scratch_bytes(int64_t B, int64_t Hq, int64_t Qb) {
  return single_pass_e_bytes(B, Hq, Qb) + B * Hq * ring_slots(Qb) * 256;
}

// A half-row block sum above this triggers the max check (the row's
// reference point is raised only when the block max exceeds it by more than
// kRescaleThreshold).
constexpr float kMassCheckSum = 256.0f;

// PASS 1: row statistics; PASS 2: tile mass from them; PASS 3: single pass
// with per-row partials in the workspace.
template <int D, int WAVES, typename TIn, bool F16, int PASS>
__global__ __launch_bounds__(WAVES * 64) void block_mass_kernel(const MassParams p) {
  constexpr int NTHR = WAVES * 64;
  constexpr int KSTR = D + 8;
  constexpr int KTILE = kBlock * KSTR;
  constexpr int KROWCH = D / 8;
  constexpr int KCHUNKS = kBlock * KROWCH;
  constexpr int KCH = (KCHUNKS + NTHR - 1) / NTHR;
  constexpr int KS = D / 16;
  constexpr int EB = TIn::bytes;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * KTILE];
  // Single pass: each wave stages its rows' e_J for kRing blocks here, all
  // relative to the row's current reference point, and copies them to the
  // scratch in one go (see flush_ring).  Slot J % kRing, row l32.
  __shared__ __attribute__((aligned(16))) float ring[PASS == 3 ? WAVES : 1][PASS == 3 ? kRing * 32 : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps per-wave addresses scalar
  const int l32 = lane & 31, hl = lane >> 5;

  const int nrows = p.B * p.Hkv * p.Qb;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int chunk = slot / p.parts;
  const int part = slot - chunk * p.parts;
  const int roww = chunk * 8 + xcd;
  if (roww >= nrows) return;
  const int bh = p.B * p.Hkv;
  const int qb = p.Qb - 1 - roww / bh;  // heaviest rows first
  const int bg = roww - (roww / bh) * bh;
  const int b = bg / p.Hkv, g = bg - (bg / p.Hkv) * p.Hkv;
  const int tile = part * p.tpp + wave;
  const bool active = wave < p.tpp && tile < 2 * p.G;
  const int hq = active ? (tile >> 1) : 0;
  const int head = g * p.G + hq;
  const int half = tile & 1;
  const int q0 = qb * kBlock + half * 32;
  const int qin = half * 32 + l32;
  const int qtok = q0 + l32;
  uint4 qf[KS];
  {
    const int qrs = (int)(p.qs[2] * EB);
    int nq = p.T - q0;
    nq = nq < 0 ? 0 : (nq > 32 ? 32 : nq);
    if (!active) nq = 0;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        static_cast<const char*>(p.q) + ((int64_t)b * p.qs[0] + (int64_t)head * p.qs[1] + (int64_t)q0 * p.qs[2]) * EB,
        (uint32_t)(nq * qrs));
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[kk] = raw_to_mfma<TIn, F16>(buf_load8<TIn>(rq, l32 * qrs + (16 * kk + 8 * hl) * EB));
  }

  const char* kbase = static_cast<const char*>(p.k) + ((int64_t)b * p.ks[0] + (int64_t)g * p.ks[1]) * EB;
  const int krs = (int)(p.ks[2] * EB);
  static_assert(NTHR % KROWCH == 0, "staging layout");
  constexpr int KRP = NTHR / KROWCH;
  const int key0 = tid / KROWCH, dc0 = tid % KROWCH;
  const int koff0 = key0 * krs + dc0 * 8 * EB, klds0 = key0 * KSTR + dc0 * 8;
  raw8_t<TIn> kst[KCH];
  auto load_k = [&](int blk) {
    int nk = p.T - blk * kBlock;
    nk = nk > kBlock ? kBlock : nk;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)blk * kBlock * krs, (uint32_t)(nk * krs));
#pragma unroll
    for (int i = 0; i < KCH; ++i)
      kst[i] = buf_load8<TIn>(rk, key0 + i * KRP < kBlock ? koff0 + i * KRP * krs : kOutOfRange);
  };
  auto store_k = [&](int buf) {
    uint16_t* Ks = smem + buf * KTILE;
#pragma unroll
    for (int i = 0; i < KCH; ++i)
      if ((KCHUNKS % NTHR) == 0 || key0 + i * KRP < kBlock)
        *reinterpret_cast<uint4*>(Ks + klds0 + i * KRP * KSTR) = raw_to_mfma<TIn, F16>(kst[i]);
  };

  // Row statistics in log2 units: m_use is the reference point, l_run the
  // running sum relative to it (pass 1 and 3 build them; pass 2 reads them).
  float m_use = 0.f, l_run = 0.f, inv_l = 0.f;
  float* stat = p.stats + (((int64_t)b * p.Hq + head) * p.T + (qtok < p.T ? qtok : 0)) * 2;
  if (PASS == 2 && active && qtok < p.T) {
    m_use = stat[0];
    inv_l = 1.f / stat[1];
  }
  float* part_out = p.part + ((((int64_t)b * p.Hq + head) * 2 + half) * p.Qb + qb) * p.Qb;
  // Single pass: this tile's e_J rows (J = 0..qb, 32 rows each) and its
  // per-ring reference points (ring r covers J = r kRing .. r kRing + kRing - 1).
  float* rowe = nullptr;
  float* rowm = nullptr;
  if (PASS == 3) {
    const int64_t tileh = ((int64_t)b * p.Hq + head) * 2 + half;
    rowe = p.rowe + (tileh * ((int64_t)p.Qb * (p.Qb + 1) / 2) + (int64_t)qb * (qb + 1) / 2) * 32;
    rowm = p.rowm + (tileh * ring_slots(p.Qb) + ring_slots(qb)) * 32;
  }

  // Copies the full ring of blocks J0..J0+kRing-1 to the scratch (16 bytes
  // per lane per store, kRing * 128 bytes contiguous) with the rows'
  // reference point.  Staging through LDS keeps the global stores to one
  // block in kRing: a store still in flight makes the next K staging wait for
  // its write acknowledgement (loads and stores share the counter and may
  // complete out of order), which per block cost about a tenth of the kernel
  // time.
  auto flush_ring = [&](int J0) {
    if constexpr (PASS == 3) {
      __builtin_amdgcn_wave_barrier();  // the ring's slots were written by the lanes of half 0
      const float4* src = reinterpret_cast<const float4*>(&ring[wave][0]);
      float4* dst = reinterpret_cast<float4*>(rowe + (int64_t)J0 * 32);
#pragma unroll
      for (int i = 0; i < kRing * 8 / 64; ++i) dst[lane + 64 * i] = src[lane + 64 * i];
      if (hl == 0) rowm[(int64_t)(J0 / kRing) * 32 + l32] = m_use;
      __builtin_amdgcn_wave_barrier();  // the copies are read before the slots are reused
    }
  };

  // One block of the row: S^T = K Q^T (from the reference point), the
  // exponentials, the row-statistics update (PASS 1/3) and the partial
  // (PASS 3) or tile mass (PASS 2).  The diagonal block (last) is the only
  // one with a causal mask, so it runs as its own instance.
  auto step = [&](auto diag_tag, int J, int buf) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const uint16_t* kp = smem + buf * KTILE + l32 * KSTR + 8 * hl;
    f32x16_t s0 = f32x16_t{}, s1 = f32x16_t{};
    uint4 a0 = *reinterpret_cast<const uint4*>(kp);
    uint4 a1 = *reinterpret_cast<const uint4*>(kp + 32 * KSTR);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      uint4 n0 = a0, n1 = a1;
      if (kk + 1 < KS) {
        n0 = *reinterpret_cast<const uint4*>(kp + 16 * (kk + 1));
        n1 = *reinterpret_cast<const uint4*>(kp + 32 * KSTR + 16 * (kk + 1));
      }
      s0 = mfma32x32x16<F16>(a0, qf[kk], s0);
      s1 = mfma32x32x16<F16>(a1, qf[kk], s1);
      a0 = n0;
      a1 = n1;
    }
    if constexpr (DIAG) {
      // Register r of key tile c holds key 32c + 8(r/4) + 4(lane/32) + r%4.
      const int thr = qin - 4 * hl;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + (r & 3);
        if (kr > thr) s0[r] = -INFINITY;
        if (32 + kr > thr) s1[r] = -INFINITY;
      }
    }
    // x = exp2(s * cs - m_use).  The sum starts from the first pair: adding
    // it to +0.0 would cost an add per element (x + 0.0 is not x for
    // x = -0.0, so the compiler keeps it).
    const float cs = p.cs, nm = -m_use;
    float ps = fast_exp2(fmaf(s0[0], cs, nm)) + fast_exp2(fmaf(s1[0], cs, nm));
#pragma unroll
    for (int r = 1; r < 16; ++r) ps += fast_exp2(fmaf(s0[r], cs, nm)) + fast_exp2(fmaf(s1[r], cs, nm));
    if (PASS == 1 || PASS == 3) {
      // Block 0 sets the reference point; later blocks only check their
      // sum (NaN / inf included) and take the max when it is large.
      if (__ballot(J == 0 || !(ps <= kMassCheckSum)) != 0) {
        float mx = fmaxf(s0[0], s0[1]);
#pragma unroll
        for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s0[r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[r]);
        mx = fmaf(half_max(mx), cs, nm);  // relative to m_use
        const float delta = (J == 0 || mx > kRescaleThreshold) ? mx : 0.f;
        if (__ballot(delta != 0.f) != 0) {
          m_use += delta;
          const float f = fast_exp2(-delta);
          l_run *= f;
          if (PASS == 3 && hl == 0 && delta != 0.f) {
            // The ring's earlier blocks move to the new reference point too.
            for (int j = 0; j < J % kRing; ++j) ring[PASS == 3 ? wave : 0][j * 32 + l32] *= f;
          }
          const float nm2 = -m_use;
          ps = fast_exp2(fmaf(s0[0], cs, nm2)) + fast_exp2(fmaf(s1[0], cs, nm2));
#pragma unroll
          for (int r = 1; r < 16; ++r) ps += fast_exp2(fmaf(s0[r], cs, nm2)) + fast_exp2(fmaf(s1[r], cs, nm2));
        }
      }
      l_run += ps;
      if (PASS == 3) {
        const float e = half_sum(ps);
        if (hl == 0) ring[PASS == 3 ? wave : 0][(J % kRing) * 32 + l32] = e;
        // A full ring goes to scratch; the row's last ring (the one holding
        // the diagonal block) stays in LDS for the readback.
        if (!DIAG && J % kRing == kRing - 1) flush_ring(J - (kRing - 1));
      }
    } else {
      float v = (qtok < p.T) ? ps * inv_l : 0.f;
      // Sum over the wave's 32 query rows x 64 keys (fixed butterfly order).
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
      if (lane == 0) part_out[J] = v;
    }
  };

  // With a wave that owns no tile (G = 3, 5, 6, 7 in 8-wave parts) and
  // 16-bit inputs, that wave stages every K block alone by loads straight
  // into LDS (17 buffer loads for the tile's padded rows, the pad granules
  // out of range) and the tile waves only compute; both sides keep the same
  // barrier sequence, and the producer leaves after the last block (no
  // barrier follows the loop).
  constexpr int KG = KSTR / 8;  // 16-byte granules per LDS row, data and pad
  const bool producer_form = EB == 2 && p.tpp < WAVES;
  if (producer_form && wave == WAVES - 1) {
    if constexpr (EB == 2) {
      int kdma[KG];
#pragma unroll
      for (int i = 0; i < KG; ++i) {
        const int gidx = 64 * i + lane, row = gidx / KG, col = gidx - row * KG;
        kdma[i] = col < KROWCH ? row * krs + col * 16 : kOutOfRange;
      }
      auto stage = [&](int blk, int sbuf) {
        int nk = p.T - blk * kBlock;
        nk = nk > kBlock ? kBlock : nk;
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)blk * kBlock * krs, (uint32_t)(nk * krs));
        uint16_t* Ks = smem + sbuf * KTILE;
#pragma unroll
        for (int i = 0; i < KG; ++i) buffer_load_lds16(rk, Ks + 512 * i, kdma[i]);
      };
      stage(0, 0);
      __syncthreads();
      int pbuf = 0;
      for (int J = 0; J < qb; ++J) {
        stage(J + 1, pbuf ^ 1);
        __syncthreads();
        pbuf ^= 1;
      }
    }
    return;
  }
  if (!producer_form) {
    load_k(0);
    store_k(0);
  }
  __syncthreads();
  int buf = 0;
  for (int J = 0; J < qb; ++J) {
    if (!producer_form) load_k(J + 1);
    if (active) step(std::false_type{}, J, buf);
    if (!producer_form) store_k(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  if (active) step(std::true_type{}, qb, buf);
  if (PASS == 1 && active) {
    const float lt = half_sum(l_run);
    if (hl == 0 && qtok < p.T) {
      stat[0] = m_use;
      stat[1] = lt;
    }
  }
  if constexpr (PASS == 3) {
    if (!active) return;
    const float lt = half_sum(l_run);
    const float inv = (qtok < p.T && lt > 0.f) ? 1.f / lt : 0.f;
    // The wave reads back only what it wrote, on the same CU: a
    // workgroup-scope fence (wait for the stores) orders them before the
    // loads.  An agent-scope fence would also write back this XCD's L2.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    __builtin_amdgcn_wave_barrier();  // the last ring's slots were written by the lanes of half 0
    // One ring (16 key blocks) per step, all loads issued first: lane half hl
    // takes J = J0 + 2u + hl (u = 0..7), lane l32 row l32; each J is then
    // summed over the 32 rows by a fixed butterfly.  Full rings come from
    // the scratch, the last one from LDS (relative to the current reference).
    constexpr int U = kRing / 2;
    const int Jlast = qb - qb % kRing;
    for (int J0 = 0; J0 <= qb; J0 += 2 * U) {
      float e[U];
      float mr = m_use;
      if (J0 < Jlast) {
        mr = rowm[(int64_t)(J0 / kRing) * 32 + l32];
#pragma unroll
        for (int u = 0; u < U; ++u) e[u] = rowe[(int64_t)(J0 + 2 * u + hl) * 32 + l32];
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int J = J0 + 2 * u + hl;
          e[u] = J <= qb ? ring[wave][(J % kRing) * 32 + l32] : 0.f;
        }
      }
      const float w = fast_exp2(mr - m_use) * inv;
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = e[u] * w;
#pragma unroll
      for (int off = 16; off >= 1; off >>= 1)
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] += __shfl_xor(v[u], off);
      if (l32 == 0) {
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (J0 + 2 * u + hl <= qb) part_out[J0 + 2 * u + hl] = v[u];
      }
    }
  }
}

// mass[b,h,I,J] = part[b,h,0,I,J] + part[b,h,1,I,J] for J <= I, 0 above.
__global__ __launch_bounds__(256) void mass_combine_kernel(const float* __restrict__ part, int64_t slabs, int Qb,
                                                           float* __restrict__ mass) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)Qb * Qb;
  if (idx >= slabs * per) return;
  const int64_t s = idx / per;
  const int64_t r = idx - s * per;
  const int I = (int)(r / Qb), J = (int)(r - (int64_t)(r / Qb) * Qb);
  const float* p0 = part + s * 2 * per;
  mass[idx] = J <= I ? p0[r] + p0[per + r] : 0.f;
}

__device__ __forceinline__ uint32_t target_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Per (batch, KV head, query block) row: mean over the group's query heads,
// causal mask, row normalisation, then the k largest targets (descending,
// ties to the lower block index; -1 padding for short causal rows).
constexpr int kTgtMaxKb = 8192;
// NORM = false: only the group mean with the causal mask (into target) and its
// row sum, for callers that normalise later.
template <bool NORM>
__global__ __launch_bounds__(256) void teacher_targets_kernel(const float* __restrict__ mass, int Hq, int Hkv,
                                                              int Qb, int Kb, int k, float eps,
                                                              float* __restrict__ target, float* __restrict__ row_mass,
                                                              int32_t* __restrict__ topk) {
  __shared__ float vals[kTgtMaxKb];
  __shared__ float red[256];
  __shared__ int hist[256];
  __shared__ int sel_bin, sel_rem;
  __shared__ int sel_idx[64];
  __shared__ uint32_t sel_key[64];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;  // (b*Hkv + g)*Qb + i
  const int i = row % Qb;
  const int bg = row / Qb;
  const int g = bg % Hkv, b = bg / Hkv;
  const int G = Hq / Hkv;
  const int n = i + 1 < Kb ? i + 1 : Kb;
  float part = 0.f;
  const int64_t hs = (int64_t)Qb * Kb;  // head stride of mass
  const float* mrow = mass + ((((int64_t)b * Hq + g * G) * Qb) + i) * Kb;
  for (int j = tid; j < Kb; j += 256) {
    float v = 0.f;
    if (j < n) {
      if (G <= 8) {
        // Every head's load is issued before the first add (heads past G
        // re-read head 0, not added); the sum is the same ordered sequence.
        float x[8];
#pragma unroll
        for (int h = 0; h < 8; ++h) x[h] = mrow[(h < G ? h : 0) * hs + j];
#pragma unroll
        for (int h = 0; h < 8; ++h)
          if (h < G) v += x[h];
      } else {
        for (int h = 0; h < G; ++h) v += mrow[h * hs + j];
      }
      v = v / (float)G;
    }
    vals[j] = v;
    part += v;
  }
  red[tid] = part;
  __syncthreads();
  for (int st = 128; st >= 1; st >>= 1) {
    if (tid < st) red[tid] += red[tid + st];
    __syncthreads();
  }
  const float rs = red[0];
  float* trow = target + (int64_t)row * Kb;
  if constexpr (!NORM) {
    for (int j = tid; j < Kb; j += 256) trow[j] = vals[j];
    if (tid == 0) row_mass[row] = rs;
    return;
  }
  const float den = rs > eps ? rs : eps;
  for (int j = tid; j < Kb; j += 256) {
    const float t = vals[j] / den;
    trow[j] = t;
    vals[j] = t;
  }
  if (tid == 0) row_mass[row] = rs;
  __syncthreads();
  int32_t* o = topk + (int64_t)row * k;
  const int m = n < k ? n : k;
  // Radix select of the m-th largest target key among the causal entries.
  uint32_t prefix = 0, mask = 0;
  int rem = m;
  for (int pass = 3; pass >= 0; --pass) {
    hist[tid] = 0;
    __syncthreads();
    const int sh = 8 * pass;
    for (int j = tid; j < n; j += 256) {
      const uint32_t key = target_key(vals[j]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> sh) & 255], 1);
    }
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
  if (tid < 64) {
    int eq_base = 0, out_base = 0;
    const uint64_t lt = (tid == 0) ? 0ull : (~0ull >> (64 - tid));
    for (int c0 = 0; c0 < n; c0 += 64) {
      const int j = c0 + tid;
      const uint32_t key = j < n ? target_key(vals[j]) : 0u;
      const bool eq = j < n && key == prefix;
      const uint64_t eqb = __ballot(eq);
      const int rank = eq_base + __popcll(eqb & lt);
      const bool sel = j < n && (key > prefix || (eq && rank < rem));
      const uint64_t sb = __ballot(sel);
      if (sel) {
        const int pos = out_base + __popcll(sb & lt);
        sel_idx[pos] = j;
        sel_key[pos] = key;
      }
      eq_base += __popcll(eqb);
      out_base += __popcll(sb);
    }
    // Order the m selected entries by target descending, index ascending.
    if (tid < m) {
      const uint32_t key = sel_key[tid];
      const int idx = sel_idx[tid];
      int rank = 0;
      for (int t = 0; t < m; ++t) rank += (sel_key[t] > key) || (sel_key[t] == key && sel_idx[t] < idx);
      o[rank] = idx;
    }
    if (tid >= m && tid < k) o[tid] = -1;
  }
}

// Rows of at most 256 key blocks: one wavefront per row, entries j = lane +
// 64 s (s < 4) in registers, no LDS staging of the row and no workgroup
// barrier.  Results are those of teacher_targets_kernel bit for bit: the row
// sum follows its 256-entry reduction tree (entries j and j + 128, then j and
// j + 64, inside each lane; then lanes l and l + s for s = 32 .. 1), and the
// top-k takes the same entries (every key above the m-th largest key T, then
// the lowest-index keys equal to T) in the same order.
constexpr int kTgtWaveKb = 256;

template <bool NORM>
__global__ __launch_bounds__(256) void teacher_targets_wave_kernel(const float* __restrict__ mass, int Hq, int Hkv,
                                                                   int Qb, int Kb, int k, float eps, int rows,
                                                                   float* __restrict__ target,
                                                                   float* __restrict__ row_mass,
                                                                   int32_t* __restrict__ topk) {
  __shared__ int sel_idx[4][64];
  __shared__ uint32_t sel_key[4][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int row = blockIdx.x * 4 + w;
  if (row >= rows) return;  // uniform per wave; the kernel has no workgroup barrier
  const int i = row % Qb;
  const int bg = row / Qb;
  const int g = bg % Hkv, b = bg / Hkv;
  const int G = Hq / Hkv;
  const int n = i + 1 < Kb ? i + 1 : Kb;
  const int64_t hs = (int64_t)Qb * Kb;
  const float* mrow = mass + ((((int64_t)b * Hq + g * G) * Qb) + i) * Kb;

  // Group mean; every load is issued before the first add (entries past the
  // causal range and heads past G re-read an entry in range, not added).
  float v[4];
  if (G <= 8) {
    float x[4][8];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int j = lane + 64 * s4;
      const int jc = j < n ? j : n - 1;
#pragma unroll
      for (int h = 0; h < 8; ++h) x[s4][h] = mrow[(h < G ? h : 0) * hs + jc];
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      float a = 0.f;
#pragma unroll
      for (int h = 0; h < 8; ++h)
        if (h < G) a += x[s4][h];
      v[s4] = lane + 64 * s4 < n ? a / (float)G : 0.f;
    }
  } else {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int j = lane + 64 * s4;
      float a = 0.f;
      if (j < n) {
        for (int h = 0; h < G; ++h) a += mrow[h * hs + j];
        a = a / (float)G;
      }
      v[s4] = a;
    }
  }
  // Row sum in the workgroup kernel's tree order.
  float x = ((0.f + v[0]) + (0.f + v[2])) + ((0.f + v[1]) + (0.f + v[3]));
#pragma unroll
  for (int st = 32; st >= 1; st >>= 1) x = x + __shfl_down(x, st);
  const float rs = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
  float* trow = target + (int64_t)row * Kb;
  if (lane == 0) row_mass[row] = rs;
  if constexpr (!NORM) {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      if (lane + 64 * s4 < Kb) trow[lane + 64 * s4] = v[s4];
    return;
  }
  const float den = rs > eps ? rs : eps;
  uint32_t key[4];
  bool ok[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    const int j = lane + 64 * s4;
    const float t = v[s4] / den;
    if (j < Kb) trow[j] = t;
    ok[s4] = j < n;
    key[s4] = target_key(t);
  }
  // T: the largest key with at least m keys at or above it (the m-th largest).
  const int m = n < k ? n : k;
  uint32_t T = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t c = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) cnt += __popcll(__ballot(ok[s4] && key[s4] >= c));
    if (cnt >= m) T = c;
  }
  int above = 0;
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) above += __popcll(__ballot(ok[s4] && key[s4] > T));
  const int rem = m - above;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int eq_base = 0, out_base = 0;
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    const int j = lane + 64 * s4;
    const bool eq = ok[s4] && key[s4] == T;
    const uint64_t eqb = __ballot(eq);
    const int rank = eq_base + __popcll(eqb & lt);
    const bool sel = ok[s4] && (key[s4] > T || (eq && rank < rem));
    const uint64_t sb = __ballot(sel);
    if (sel) {
      const int pos = out_base + __popcll(sb & lt);
      sel_idx[w][pos] = j;
      sel_key[w][pos] = key[s4];
    }
    eq_base += __popcll(eqb);
    out_base += __popcll(sb);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Order the m selected entries by target descending, index ascending.
  int32_t* o = topk + (int64_t)row * k;
  if (lane < m) {
    const uint32_t kk = sel_key[w][lane];
    const int idx = sel_idx[w][lane];
    int r = 0;
    for (int t = 0; t < m; ++t) r += (sel_key[w][t] > kk) || (sel_key[w][t] == kk && sel_idx[w][t] < idx);
    o[r] = idx;
  }
  if (lane >= m && lane < k) o[lane] = -1;
}

template <int D, typename TIn, bool F16, int PASS>
int launch_mass_w(const MassParams& p, int waves, hipStream_t s) {
  const int64_t grid = ((int64_t)p.B * p.Hkv * p.Qb + 7) / 8 * 8 * p.parts;
  switch (waves) {
    case 2: hipLaunchKernelGGL((block_mass_kernel<D, 2, TIn, F16, PASS>), dim3((unsigned)grid), dim3(128), 0, s, p); break;
    case 4: hipLaunchKernelGGL((block_mass_kernel<D, 4, TIn, F16, PASS>), dim3((unsigned)grid), dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL((block_mass_kernel<D, 8, TIn, F16, PASS>), dim3((unsigned)grid), dim3(512), 0, s, p); break;
    default: return set_error(SPRUCE_EINVAL, "unsupported wave count %d", waves);
  }
  return check_launch("block_mass_kernel");
}

// Bytes of the per-half tile partials [B, Hq, 2, Qb, Qb] float32, 256-byte rounded.
inline size_t part_bytes(int64_t B, int64_t Hq, int64_t Qb) {
  return ((size_t)B * Hq * 2 * Qb * Qb * sizeof(float) + 255) / 256 * 256;
}

// Workspace of each schedule.
inline size_t schedule_workspace_bytes(int64_t B, int64_t Hq, int64_t T, int schedule) {
  const int64_t Qb = (T + kBlock - 1) / kBlock;
  switch (schedule) {
    case SPRUCE_TEACHER_SCRATCH: return part_bytes(B, Hq, Qb) + (size_t)single_pass_scratch_bytes(B, Hq, Qb);
    default: return (size_t)(B * Hq * T * 2 + B * Hq * 2 * Qb * Qb) * sizeof(float);
  }
}

template <int PASS>
int launch_mass(const MassParams& p, int D, int dtype, int waves, hipStream_t s) {
  if (D == 128) {
    if (dtype == SPRUCE_DTYPE_BF16) return launch_mass_w<128, InBF16, false, PASS>(p, waves, s);
    if (dtype == SPRUCE_DTYPE_F16) return launch_mass_w<128, InF16, true, PASS>(p, waves, s);
    return launch_mass_w<128, InF32, false, PASS>(p, waves, s);
  }
  if (dtype == SPRUCE_DTYPE_BF16) return launch_mass_w<64, InBF16, false, PASS>(p, waves, s);
  if (dtype == SPRUCE_DTYPE_F16) return launch_mass_w<64, InF16, true, PASS>(p, waves, s);
  return launch_mass_w<64, InF32, false, PASS>(p, waves, s);
}

}  // namespace spruce

using namespace spruce;

namespace {

// Schedule of the auto mode: the single pass when its scratch is at most
// kSinglePassScratchMax and the workspace holds it, else two passes.
int pick_schedule(int64_t B, int64_t Hq, int64_t T, size_t workspace_bytes) {
  const int64_t Qb = (T + kBlock - 1) / kBlock;
  if (single_pass_scratch_bytes(B, Hq, Qb) <= kSinglePassScratchMax &&
      workspace_bytes >= schedule_workspace_bytes(B, Hq, T, SPRUCE_TEACHER_SCRATCH))
    return SPRUCE_TEACHER_SCRATCH;
  return SPRUCE_TEACHER_TWO_PASS;
}

}  // namespace

extern "C" int spruce_teacher_block_mass_schedule(const void* q, const int64_t qs[4], const void* k,
                                                  const int64_t ks[4], int64_t B, int64_t Hq, int64_t Hkv, int64_t T,
                                                  int64_t D, float scale, int dtype, float* mass, float* workspace,
                                                  size_t workspace_bytes, int schedule, void* stream) {
  // Reuse the attention argument checks (v aliases k; out only needs alignment).
  AttnParams ap;
  LaunchShape shape;
  const int64_t fake_os[4] = {0, 0, 4, 1};
  int rc = prepare_attention(ap, q, qs, k, ks, k, ks, B, Hq, Hkv, T, D, scale, dtype, SPRUCE_VARIANT_SINGLE_HEAD,
                             mass, fake_os, shape);
  if (rc) return rc;
  SPRUCE_REQUIRE(mass != nullptr && workspace != nullptr, "mass and workspace must be non-null");
  SPRUCE_REQUIRE(schedule >= SPRUCE_TEACHER_AUTO && schedule <= SPRUCE_TEACHER_TWO_PASS, "unknown schedule %d",
                 schedule);
  SPRUCE_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "workspace must be 16-byte aligned");
  const int64_t Qb = (T + kBlock - 1) / kBlock;
  if (schedule == SPRUCE_TEACHER_AUTO) schedule = pick_schedule(B, Hq, T, workspace_bytes);
  if (schedule == SPRUCE_TEACHER_SCRATCH)
    SPRUCE_REQUIRE(single_pass_scratch_bytes(B, Hq, Qb) <= kSinglePassScratchMax,
                   "the scratch schedule needs more than %lld bytes of scratch", (long long)kSinglePassScratchMax);
  const size_t need = schedule_workspace_bytes(B, Hq, T, schedule);
  SPRUCE_REQUIRE(workspace_bytes >= need, "workspace too small: %zu bytes, need %zu", workspace_bytes, need);
  MassParams p{};
  p.q = q;
  p.k = k;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = qs[i];
    p.ks[i] = ks[i];
  }
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.T = (int)T;
  p.G = (int)(Hq / Hkv);
  p.Qb = (int)Qb;
  p.parts = shape.parts;
  p.tpp = shape.tpp;
  p.cs = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  if (schedule == SPRUCE_TEACHER_SCRATCH) {
    // [part: B*Hq*2*Qb*Qb floats][rowe: e_J floats][rowm: m_r floats], each 256-byte aligned.
    p.part = workspace;
    p.rowe = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + part_bytes(B, Hq, Qb));
    p.rowm = reinterpret_cast<float*>(reinterpret_cast<char*>(p.rowe) + single_pass_e_bytes(B, Hq, Qb));
    rc = launch_mass<3>(p, (int)D, dtype, shape.waves, s);
    if (rc) return rc;
  } else {
    p.stats = workspace;
    p.part = workspace + (size_t)B * Hq * T * 2;
    rc = launch_mass<1>(p, (int)D, dtype, shape.waves, s);
    if (rc) return rc;
    rc = launch_mass<2>(p, (int)D, dtype, shape.waves, s);
    if (rc) return rc;
  }
  const int64_t total = B * Hq * Qb * Qb;
  hipLaunchKernelGGL(mass_combine_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, p.part, B * Hq,
                     (int)Qb, mass);
  return check_launch("mass_combine_kernel");
}

extern "C" int spruce_teacher_block_mass(const void* q, const int64_t qs[4], const void* k, const int64_t ks[4],
                                         int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D, float scale,
                                         int dtype, float* mass, float* workspace, size_t workspace_bytes,
                                         void* stream) {
  return spruce_teacher_block_mass_schedule(q, qs, k, ks, B, Hq, Hkv, T, D, scale, dtype, mass, workspace,
                                            workspace_bytes, SPRUCE_TEACHER_AUTO, stream);
}

extern "C" int spruce_teacher_schedule(int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
                                       size_t workspace_bytes) {
  SPRUCE_REQUIRE(B >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 && T >= 1 && (D == 64 || D == 128),
                 "invalid shape");
  return pick_schedule(B, Hq, T, workspace_bytes);
}

extern "C" size_t spruce_teacher_schedule_workspace_bytes(int64_t B, int64_t Hq, int64_t T, int schedule) {
  if (B < 1 || Hq < 1 || T < 1) return 0;
  if (schedule == SPRUCE_TEACHER_AUTO) {
    const int64_t Qb = (T + kBlock - 1) / kBlock;
    schedule = single_pass_scratch_bytes(B, Hq, Qb) <= kSinglePassScratchMax ? SPRUCE_TEACHER_SCRATCH
                                                                               : SPRUCE_TEACHER_TWO_PASS;
  }
  return schedule_workspace_bytes(B, Hq, T, schedule);
}

extern "C" size_t spruce_teacher_workspace_bytes_min(int64_t B, int64_t Hq, int64_t T) {
  return schedule_workspace_bytes(B, Hq, T, SPRUCE_TEACHER_TWO_PASS);
}

extern "C" size_t spruce_teacher_workspace_bytes(int64_t B, int64_t Hq, int64_t T) {
  return spruce_teacher_schedule_workspace_bytes(B, Hq, T, SPRUCE_TEACHER_AUTO);
}

extern "C" int spruce_teacher_targets(const float* mass, int64_t B, int64_t Hq, int64_t Hkv, int64_t Qb, int64_t Kb,
                                      int64_t k, float eps, float* target, float* row_mass, int32_t* topk,
                                      void* stream) {
  SPRUCE_REQUIRE(mass && target && row_mass && topk, "mass, target, row_mass and topk must be non-null");
  SPRUCE_REQUIRE(B >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 && Qb >= 1 && Kb >= 1, "invalid shape");
  SPRUCE_REQUIRE(k >= 1 && k <= 64, "k must be in [1, 64], got %lld", (long long)k);
  SPRUCE_REQUIRE(Kb <= kTgtMaxKb, "at most %d key blocks per row are supported", kTgtMaxKb);
  SPRUCE_REQUIRE(B * Hkv * Qb < ((int64_t)1 << 31), "too many rows");
  const int64_t rows = B * Hkv * Qb;
  if (Kb <= kTgtWaveKb) {
    hipLaunchKernelGGL(teacher_targets_wave_kernel<true>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, mass, (int)Hq, (int)Hkv, (int)Qb, (int)Kb, (int)k, eps, (int)rows, target,
                       row_mass, topk);
    return check_launch("teacher_targets_wave_kernel");
  }
  hipLaunchKernelGGL(teacher_targets_kernel<true>, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                     mass, (int)Hq, (int)Hkv, (int)Qb, (int)Kb, (int)k, eps, target, row_mass, topk);
  return check_launch("teacher_targets_kernel");
}

extern "C" int spruce_teacher_group_mass(const float* mass, int64_t B, int64_t Hq, int64_t Hkv, int64_t Qb,
                                         int64_t Kb, float* group_mass, float* row_mass, void* stream) {
  SPRUCE_REQUIRE(mass && group_mass && row_mass, "mass, group_mass and row_mass must be non-null");
  SPRUCE_REQUIRE(B >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 && Qb >= 1 && Kb >= 1, "invalid shape");
  SPRUCE_REQUIRE(Kb <= kTgtMaxKb, "at most %d key blocks per row are supported", kTgtMaxKb);
  SPRUCE_REQUIRE(B * Hkv * Qb < ((int64_t)1 << 31), "too many rows");
  const int64_t rows = B * Hkv * Qb;
  if (Kb <= kTgtWaveKb) {
    hipLaunchKernelGGL(teacher_targets_wave_kernel<false>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, mass, (int)Hq, (int)Hkv, (int)Qb, (int)Kb, 0, 0.f, (int)rows, group_mass,
                       row_mass, nullptr);
    return check_launch("teacher_targets_wave_kernel");
  }
  hipLaunchKernelGGL(teacher_targets_kernel<false>, dim3((unsigned)rows), dim3(256), 0,
                     (hipStream_t)stream, mass, (int)Hq, (int)Hkv, (int)Qb, (int)Kb, 0, 0.f, group_mass, row_mass,
                     nullptr);
  return check_launch("teacher_targets_kernel");
}
