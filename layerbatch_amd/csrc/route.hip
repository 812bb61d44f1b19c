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
#include "route_token.hpp"

namespace lbmoe {

template <int EPL>
__global__ __launch_bounds__(256) void route_topk(const uint16_t* __restrict__ logits,
                                                  const float* __restrict__ bias,
                                                  const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w_sg, int T,
                                                  int E, int H, int k, void* idx_out,
                                                  int idx_bytes, uint16_t* __restrict__ topw,
                                                  float* __restrict__ sgate,
                                                  uint8_t* __restrict__ xq,
                                                  float* __restrict__ xs) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_token<EPL>(logits, bias, x, w_sg, t, E, H, k, idx_out, idx_bytes, topw, sgate, xq, xs);
}

hipError_t launch_route_topk(const void* logits, const float* bias, const void* x,
                             const void* w_sg, int64_t T, int E, int H, int k, void* idx,
                             int idx_bytes, void* topw, float* sgate, hipStream_t s, void* xq,
                             float* xs) {
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  const auto* lg = static_cast<const uint16_t*>(logits);
  const auto* xx = static_cast<const uint16_t*>(x);
  const auto* ws = static_cast<const uint16_t*>(w_sg);
  auto* tw = static_cast<uint16_t*>(topw);
  const int Ti = static_cast<int>(T);
#define LBMOE_ROUTE(EPL)                                                                       \
  route_topk<EPL><<<grid, 256, 0, s>>>(lg, bias, xx, ws, Ti, E, H, k, idx, idx_bytes, tw, sgate, \
                                       static_cast<uint8_t*>(xq), xs)
  if (E <= 64) LBMOE_ROUTE(1);
  else if (E <= 128) LBMOE_ROUTE(2);
  else if (E <= 256) LBMOE_ROUTE(4);
  else if (E <= 512) LBMOE_ROUTE(8);
  else LBMOE_ROUTE(16);
#undef LBMOE_ROUTE
  return hipGetLastError();
}

}  // namespace lbmoe
