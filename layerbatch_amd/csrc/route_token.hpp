// One token's router selection, executed by one wave: softmax -> top-k -> renormalise -> bf16
// and the shared-expert gate (the algorithm and its reference lines are described in
// route.hip). Shared by the route kernel and the fused route + permutation kernel of small
// batches.
#pragma once

#include <float.h>

#include "common.hpp"

namespace lbmoe {

// Order-preserving map float -> uint32 (larger float -> larger key); -0 maps with +0.
__device__ __forceinline__ uint32_t order_key(float z) {
  const uint32_t u = __float_as_uint(z + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave-wide maximum of v (DPP within each 16-lane row, then the four row maxima).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xf, 0xf, false)));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}
__device__ __forceinline__ int wave_min_i32(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xf, 0xf, false));
  const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return min(min(r0, r1), min(r2, r3));
}

// Token t's selection: idx_out[t*k + s] (idx_bytes 4 or 8), topw[t*k + s] and sgate[t] (each
// when not null). Every lane of the wave must call it; it uses no LDS and no barrier.
template <int EPL>
__device__ __forceinline__ void route_token(const uint16_t* __restrict__ logits,
                                            const float* __restrict__ bias,
                                            const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ w_sg, int t, int E,
                                            int H, int k, void* idx_out, int idx_bytes,
                                            uint16_t* __restrict__ topw,
                                            float* __restrict__ sgate) {
  const int lane = lane_id();
  const uint16_t* lrow = logits + static_cast<int64_t>(t) * E;
  float z[EPL];
  uint32_t key[EPL];
  float m = -INFINITY;
  // unconditional loads (lanes past E read expert E-1 and are masked): a load under a
  // condition would make the compiler wait for it before the next one is issued
  uint16_t lv[EPL];
  float bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = min(j * kWave + lane, E - 1);
    lv[j] = lrow[e];
    bv[j] = bias ? bias[e] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    float v = bf2f(lv[j]) + bv[j];
    if (!(v == v) || e >= E) v = -INFINITY;   // a NaN logit is never preferred
    z[j] = v;
    key[j] = e < E ? order_key(v) : 0u;       // 0 is below every valid key
    m = fmaxf(m, v);
  }
  // the shared-expert gate, its loads in flight together with the logits'
  if (sgate != nullptr) {
    const uint16_t* xr = x + static_cast<int64_t>(t) * H;
    float d = 0.f;
    for (int c = lane * 8; c < H; c += kWave * 8) {
      const u32x4 a = ld16(xr + c);
      const u32x4 b = ld16(w_sg + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        d += bf_lo(a[q]) * bf_lo(b[q]);
        d += bf_hi(a[q]) * bf_hi(b[q]);
      }
    }
    d = round_bf(wave_sum(d));
    if (lane == 0) sgate[t] = 1.0f / (1.0f + expf(-d));
  }
  m = wave_max(m);
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    if (j * kWave + lane < E) part += expf(z[j] - m);
  const float S = wave_sum(part);

  // k rounds of argmax; lane r < k keeps round r's winner (expert and key)
  int my_e = 0;
  uint32_t my_key = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t best = key[0];
    int bj = 0;
#pragma unroll
    for (int j = 1; j < EPL; ++j)
      if (key[j] > best) {
        best = key[j];
        bj = j;
      }
    const uint32_t wmax = wave_max_u32(best);
    const uint64_t holders = __ballot(best == wmax);
    int win;                                            // winning expert
    if (__popcll(holders) == 1) {
      const int wl = __builtin_ctzll(holders);
      win = __builtin_amdgcn_readlane(bj * kWave + lane, wl);
    } else {
      win = wave_min_i32(best == wmax ? bj * kWave + lane : 0x7fffffff);
    }
    const int wj = win / kWave, wl = win % kWave;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (j == wj && lane == wl) key[j] = 0u;
    if (lane == r) {
      my_e = win;
      my_key = wmax;
    }
  }
  float p = 0.f;
  if (lane < k) {
    const uint32_t u = (my_key & 0x80000000u) ? (my_key & 0x7fffffffu) : ~my_key;   // key -> z
    p = expf(__uint_as_float(u) - m) / S;
  }
  const float psum = wave_sum(p);
  if (lane < k) {
    const int64_t o = static_cast<int64_t>(t) * k + lane;
    if (topw != nullptr) topw[o] = static_cast<uint16_t>(f2bf(p / psum));
    if (idx_bytes == 8) reinterpret_cast<int64_t*>(idx_out)[o] = my_e;
    else reinterpret_cast<int32_t*>(idx_out)[o] = my_e;
  }
}

}  // namespace lbmoe
