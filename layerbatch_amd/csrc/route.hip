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
// One wave per token; each lane holds experts lane, lane+64, ... in registers.
#include <float.h>

#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

template <int EPL>
__global__ __launch_bounds__(256) void route_topk(const uint16_t* __restrict__ logits,
                                                  const float* __restrict__ bias,
                                                  const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w_sg, int T,
                                                  int E, int H, int k, void* idx_out,
                                                  int idx_bytes, uint16_t* __restrict__ topw,
                                                  float* __restrict__ sgate) {
  const int lane = lane_id();
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* lrow = logits + static_cast<int64_t>(t) * E;
  float z[EPL];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    float v = -INFINITY;
    if (e < E) {
      v = bf2f(lrow[e]);
      if (bias) v += bias[e];
      if (!(v == v)) v = -INFINITY;     // a NaN logit is never preferred
    }
    z[j] = v;
    m = fmaxf(m, v);
  }
  m = wave_max(m);
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    if (j * kWave + lane < E) part += expf(z[j] - m);
  const float S = wave_sum(part);

  uint32_t taken = 0;
  float my_p = 0.f, psum = 0.f;
  int my_e = 0;
  for (int i = 0; i < k; ++i) {
    float bz = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = j * kWave + lane;
      if (e < E && !((taken >> j) & 1u) && (z[j] > bz || (z[j] == bz && e < be))) {
        bz = z[j];
        be = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float oz = __shfl_xor(bz, o, kWave);
      const int oe = __shfl_xor(be, o, kWave);
      if (oz > bz || (oz == bz && oe < be)) {
        bz = oz;
        be = oe;
      }
    }
    if ((be & (kWave - 1)) == lane) taken |= 1u << (be / kWave);
    const float p = expf(bz - m) / S;
    psum += p;
    if (lane == i) {
      my_p = p;
      my_e = be;
    }
  }
  if (lane < k) {
    const int64_t o = static_cast<int64_t>(t) * k + lane;
    topw[o] = static_cast<uint16_t>(f2bf(my_p / psum));
    if (idx_bytes == 8) reinterpret_cast<int64_t*>(idx_out)[o] = my_e;
    else reinterpret_cast<int32_t*>(idx_out)[o] = my_e;
  }
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
