// Device-side helpers shared by every lbmoe kernel (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbmoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// ---- bf16 ------------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even float -> bf16 bits; NaN -> canonical quiet NaN.
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return f2bf(lo) | (f2bf(hi) << 16);
}
// Value of f after rounding to bf16.
__device__ __forceinline__ float round_bf(float f) { return __uint_as_float(f2bf(f) << 16); }

// ---- OCP e4m3fn ----------------------------------------------------------------------------
// Round-to-nearest-even, saturating to +-448; NaN -> 0x7f. Values are quantised from
// x / scale with |x / scale| <= 448 up to rounding, so saturation only trims ulps.
__device__ __forceinline__ uint32_t f2e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  float a = fabsf(f);
  if (!(a == a)) return 0x7fu;
  if (a >= 448.0f) return sign | 0x7eu;
  uint32_t ua = __float_as_uint(a);
  int e = static_cast<int>(ua >> 23) - 127;              // unbiased exponent of a
  uint32_t code;
  if (e < -6) {
    // subnormal range: value = m * 2^-9, m in [0,8]; RNE of a * 2^9
    float m = a * 512.0f;                                // exact (power-of-two scale)
    float r = rintf(m);                                  // round half to even
    code = static_cast<uint32_t>(r);                     // 8 -> 0x08 = smallest normal
  } else {
    // normal: keep 3 mantissa bits with RNE on the fp32 mantissa
    uint32_t mant = ua & 0x7fffffu;
    uint32_t keep = mant >> 20;
    uint32_t rest = mant & 0xfffffu;
    uint32_t half = 0x80000u;
    uint32_t q = (static_cast<uint32_t>(e + 7) << 3) | keep;
    if (rest > half || (rest == half && (keep & 1u))) q += 1;  // carry may bump exponent
    code = q;
    if (code > 0x7eu) code = 0x7eu;
  }
  return sign | code;
}

__device__ __forceinline__ float e4m3_to_f(uint32_t c) {
  uint32_t s = c & 0x80u, e = (c >> 3) & 0xfu, m = c & 7u;
  float v = (e == 0) ? static_cast<float>(m) * (1.0f / 512.0f)
                     : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

// ---- wave reductions --------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Number of set bits of a 64-bit lane mask below this lane.
__device__ __forceinline__ int mask_rank(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// silu(g) = g / (1 + e^-g) with the hardware reciprocal (v_rcp_f32, about 1 ulp): the result
// is rounded to bf16 (or quantised to e4m3) right after, far coarser than the rcp error.
__device__ __forceinline__ float silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

}  // namespace lbmoe
