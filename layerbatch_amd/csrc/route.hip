// Router selection: softmax -> top-k -> renormalise -> bf16, and the shared-expert gate.
//
// Follows Qwen3_5TopKRouter.forward (nanovllm/models/qwen3_5.py:770-774): the bf16 logits are
// upcast to fp32 (plus an optional fp32 bias), probabilities p = exp(z - max) / sum, the k
// largest are taken and divided by their sum, then cast to bf16. torch.topk's order among
// equal probabilities is implementation-defined; here experts are ordered by descending z
// with ties broken by ascending expert index (softmax is increasing in z, so this is the
// order of descending p).
// The shared-expert gate sigmoid(x . w_sg) follows qwen3_5.py:897, :903 with the dot product
// rounded to bf16 as F.linear's bf16 output is.
//
// One wave per token; lane l holds experts l, l+64, ... in registers as order-preserving
// 32-bit keys of z. Selection is k rounds of argmax: each lane keeps its best remaining key
// (ties to the lower expert), the wave maximum comes from a DPP reduction within 16-lane rows
// and four lane reads, and the winner is the lane holding that key (on a tie between lanes,
// the lowest expert index). Round r's winner is slot r, so the slots come out in the required
// order, and the winner's key is removed. Most of the work is vector ALU; the scalar unit,
// which a CU's waves share, only combines the four row maxima.
#include <float.h>

#include "common.hpp"
#include "internal.hpp"

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

template <int EPL>
__global__ __launch_bounds__(256) void route_topk(const uint16_t* __restrict__ logits,
                                                  const float* __restrict__ bias,
                                                  const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w_sg, int T,
                                                  int E, int H, int k, void* idx_out,
                                                  int idx_bytes, uint16_t* __restrict__ topw,
                                                  float* __restrict__ sgate) {
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
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
    topw[o] = static_cast<uint16_t>(f2bf(p / psum));
    if (idx_bytes == 8) reinterpret_cast<int64_t*>(idx_out)[o] = my_e;
    else reinterpret_cast<int32_t*>(idx_out)[o] = my_e;
  }
}

hipError_t launch_route_topk(const void* logits, const float* bias, const void* x,
                             const void* w_sg, int64_t T, int E, int H, int k, void* idx,
                             int idx_bytes, void* topw, float* sgate, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  const auto* lg = static_cast<const uint16_t*>(logits);
  const auto* xx = static_cast<const uint16_t*>(x);
  const auto* ws = static_cast<const uint16_t*>(w_sg);
  auto* tw = static_cast<uint16_t*>(topw);
  const int Ti = static_cast<int>(T);
#define LBMOE_ROUTE(EPL)                                                                       \
  route_topk<EPL><<<grid, 256, 0, s>>>(lg, bias, xx, ws, Ti, E, H, k, idx, idx_bytes, tw, sgate)
  if (E <= 64) LBMOE_ROUTE(1);
  else if (E <= 128) LBMOE_ROUTE(2);
  else if (E <= 256) LBMOE_ROUTE(4);
  else if (E <= 512) LBMOE_ROUTE(8);
  else LBMOE_ROUTE(16);
#undef LBMOE_ROUTE
  return hipGetLastError();
}

}  // namespace lbmoe
