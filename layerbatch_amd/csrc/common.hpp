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

// Round-to-nearest-even float -> bf16 bits with v_cvt_pk_bf16_f32 (denormals kept; a NaN stays
// a quiet NaN with its payload's top bits). The conversion of every non-NaN float equals the
// textbook rounding (add 0x7fff plus the kept lowest bit, drop 16 bits): checked on the GPU
// over every 997th fp32 bit pattern, all halfway cases and the denormals.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
// Value of f after rounding to bf16.
__device__ __forceinline__ float round_bf(float f) { return __uint_as_float(f2bf(f) << 16); }

// ---- OCP e4m3fn ----------------------------------------------------------------------------
// Round-to-nearest-even (v_cvt_pk_fp8_f32), subnormals included. Values are quantised from
// x / scale with scale = amax / 448, so |x / scale| exceeds 448 by at most rounding and rounds
// to +-448. Four values -> four codes, a in the low byte.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// Maximum over the 16 lanes of a DPP row (lanes 16j .. 16j+15): quad permutations, then the
// half-row and row mirrors.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xb1>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4e>(v));    // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));   // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));   // row_mirror
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0xb1>(v);
  v += dpp_f32<0x4e>(v);
  v += dpp_f32<0x141>(v);
  return v + dpp_f32<0x140>(v);
}
__device__ __forceinline__ float lane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Wave-wide maximum and sum on DPP (the 16-lane row reductions above, then the four row
// results read from lanes 0, 16, 32, 48): a few cycles per step where a shuffle through LDS
// takes a round trip. Every lane of the wave must be active. The sum adds in another order
// than wave_sum.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row16_sum(v);
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

// Activation quantisation (per row and 128 channels): scale = amax / 448, 1 for an all-zero
// group; code = e4m3(value / scale). One group is held by 16 consecutive lanes of a wave
// (lanes 16j .. 16j+15, one DPP row), 8 channels per lane as 8 bf16 in v; every lane of the
// group must be active. Returns the lane's 8 codes; s receives the group's scale.
__device__ __forceinline__ float fp8_scale_of(float amax) { return amax > 0.f ? amax / 448.0f : 1.0f; }
__device__ __forceinline__ u32x2 quant_group16(u32x4 v, float& s) {
  float x[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = bf_lo(v[j]);
    x[2 * j + 1] = bf_hi(v[j]);
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
  amax = row16_max(amax);
  s = fp8_scale_of(amax);
  // x / s rounded as the division rounds it, with one division per group instead of per value
  // (Markstein): y = RN(1/s); q = RN(x y) is within an ulp of x / s, r = fma(-q, s, x) is exact
  // and RN(q + r y) = RN(x / s) while nothing underflows. Quotients under 2^-12, where r may
  // underflow, still land below e4m3's smallest step, so the codes agree; the sign is taken
  // from x (the sequence turns -0 into +0). Checked against the division on 5e8 bf16 values
  // and adversarial pairs (float32, fma, no contraction). Groups with s < 2^-80 divide, and
  // so do groups with s > 2^100 (an infinite value makes s infinite and y zero, where r would
  // be 0 * inf).
  float q[8];
  if (s >= 0x1p-80f && s <= 0x1p+100f) {
    const float y = 1.0f / s;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q0 = x[j] * y;
      q[j] = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, s, x[j]), y, q0), x[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = x[j] / s;
  }
  u32x2 c;
#pragma unroll
  for (int h = 0; h < 2; ++h) c[h] = e4m3x4(q[4 * h], q[4 * h + 1], q[4 * h + 2], q[4 * h + 3]);
  return c;
}

// ---- wave reductions --------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
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

// Stable in-wave match: the lanes of m whose value e (below 2^nbits) equals this lane's, one
// ballot per bit. With mask_rank, lanes of equal value get consecutive ranks in lane order.
__device__ __forceinline__ uint64_t match_expert(int e, uint64_t m, int nbits) {
  for (int b = 0; b < nbits; ++b) {
    const bool on = (e >> b) & 1;
    const uint64_t bal = __ballot(on);
    m &= on ? bal : ~bal;
  }
  return m;
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


// Expert id i of a routing table of int32 (IB = 4) or int64 (IB = 8) entries.
template <int IB>
__device__ __forceinline__ int load_expert(const void* idx, int64_t i) {
  if constexpr (IB == 8) return static_cast<int>(reinterpret_cast<const int64_t*>(idx)[i]);
  else return reinterpret_cast<const int32_t*>(idx)[i];
}

}  // namespace lbmoe
