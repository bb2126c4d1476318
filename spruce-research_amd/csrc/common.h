// Shared device helpers and host-side error plumbing for libspruce_hip.so.
// gfx950 (CDNA4) only: 64-lane wavefronts, 32x32x16 bf16/f16 MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/spruce_hip.h"

namespace spruce {

// ---------------------------------------------------------------- host side
// Records a formatted message in the calling thread's error slot.
int set_error(int code, const char* fmt, ...);
// Converts a launch status into the ABI return code (0 or positive hipError_t).
int check_launch(const char* what);

#define SPRUCE_REQUIRE(cond, ...)                          \
  do {                                                     \
    if (!(cond)) return ::spruce::set_error(SPRUCE_EINVAL, __VA_ARGS__); \
  } while (0)

// ------------------------------------------------------------- device types
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Element-type tags of the tensors a kernel reads.
struct InBF16 { static constexpr int code = SPRUCE_DTYPE_BF16; static constexpr int bytes = 2; };
struct InF16  { static constexpr int code = SPRUCE_DTYPE_F16;  static constexpr int bytes = 2; };
struct InF32  { static constexpr int code = SPRUCE_DTYPE_F32;  static constexpr int bytes = 4; };

// Packs two floats into one 32-bit word of two bf16 (round to nearest even,
// v_cvt_pk_bf16_f32) or two f16.
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (F16) {
    f16x2_t h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
  } else {
    f32x2_t f = {a, b};
    bf16x2_t h = __builtin_convertvector(f, bf16x2_t);
    return __builtin_bit_cast(uint32_t, h);
  }
}

// Unpacks one 16-bit value (bf16 or f16 bits) to float.
template <bool F16>
__device__ __forceinline__ float unpack1(uint32_t bits16) {
  if constexpr (F16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  } else {
    return __builtin_bit_cast(float, bits16 << 16);
  }
}

// D(32x32, fp32) += A(32x16) * B(16x32) on the matrix cores.
// Lane l supplies A row (l % 32) and B column (l % 32); the eight 16-bit
// values per lane are the k positions (l / 32) * 8 + [0, 8).
template <bool F16>
__device__ __forceinline__ f32x16_t mfma32x32x16(uint4 a, uint4 b, f32x16_t c) {
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x of lane l combined with x of lane l ^ 32, without the LDS round trip of a
// ds_bpermute: v_permlane32_swap(a, b) exchanges the upper half of a with the
// lower half of b, so with a = b = x every lane holds x[l] in one result and
// x[l ^ 32] in the other.  Both combinations are commutative, so the result
// equals x + __shfl_xor(x, 32) (resp. fmaxf) bit for bit.  (Each result is
// read into an unsigned before any bit cast: a bit cast of the vector element
// itself compiles to a read of element 0.)
__device__ __forceinline__ void half_swap(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float half_sum(float x) {
  float a, b;
  half_swap(x, a, b);
  return a + b;
}
__device__ __forceinline__ float half_max(float x) {
  float a, b;
  half_swap(x, a, b);
  return fmaxf(a, b);
}

// Maximum of v over the 64 lanes, in every lane: prefix maxima within each
// 16-lane row by DPP row shifts (lanes shifted in from outside the row keep
// their own value), then row 0's and row 2's last lanes broadcast into rows
// 1 and 3 and lane 31 into rows 2 and 3, so lane 63 holds the wave maximum.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  v = mx(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = mx(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = mx(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = mx(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = mx(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = mx(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Loads 8 consecutive elements of type TIn at p and returns them as eight
// 16-bit MFMA inputs (bf16 bits, or f16 bits when F16).  Out-of-range rows are
// handled by the caller (valid == false returns zeros).
template <typename TIn, bool F16>
__device__ __forceinline__ uint4 load8(const void* p, bool valid, float mul, bool scaled) {
  uint4 r = {0u, 0u, 0u, 0u};
  if (!valid) return r;
  if constexpr (TIn::bytes == 2) {
    r = *reinterpret_cast<const uint4*>(p);
    if (scaled) {
      uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float lo = unpack1<F16>(w[i] & 0xffffu) * mul;
        float hi = unpack1<F16>(w[i] >> 16) * mul;
        w[i] = pack2<F16>(lo, hi);
      }
      r = uint4{w[0], w[1], w[2], w[3]};
    }
  } else {
    const float4* f = reinterpret_cast<const float4*>(p);
    float4 a = f[0], b = f[1];
    if (scaled) {
      a.x *= mul; a.y *= mul; a.z *= mul; a.w *= mul;
      b.x *= mul; b.y *= mul; b.z *= mul; b.w *= mul;
    }
    r.x = pack2<F16>(a.x, a.y);
    r.y = pack2<F16>(a.z, a.w);
    r.z = pack2<F16>(b.x, b.y);
    r.w = pack2<F16>(b.z, b.w);
  }
  return r;
}

// Loads 8 consecutive elements (bf16, f16 or f32 per dtype) starting at
// element offset elem of base, widened to float.
__device__ __forceinline__ void load8f(const void* base, int64_t elem, int dtype, float* out) {
  if (dtype == SPRUCE_DTYPE_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    const float4 a = p[0], b = p[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    const bool f16 = dtype == SPRUCE_DTYPE_F16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = f16 ? unpack1<true>(w[i] & 0xffffu) : unpack1<false>(w[i] & 0xffffu);
      out[2 * i + 1] = f16 ? unpack1<true>(w[i] >> 16) : unpack1<false>(w[i] >> 16);
    }
  }
}

}  // namespace spruce
