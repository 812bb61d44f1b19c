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
// One wave per token; lane l holds experts l, l+64, ... in registers. Selection is a radix
// select on order-preserving 32-bit keys of z: 32 ballot rounds find the k-th largest key
// (no cross-lane shuffles), equal keys at the threshold are taken in ascending expert index,
// and the k winners are ranked against each other through LDS.
#include <float.h>

#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

// Order-preserving map float -> uint32 (larger float -> larger key); -0 maps with +0.
__device__ __forceinline__ uint32_t order_key(float z) {
  const uint32_t u = __float_as_uint(z + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kMaxK = 32;

template <int EPL>
__global__ __launch_bounds__(256) void route_topk(const uint16_t* __restrict__ logits,
                                                  const float* __restrict__ bias,
                                                  const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w_sg, int T,
                                                  int E, int H, int k, void* idx_out,
                                                  int idx_bytes, uint16_t* __restrict__ topw,
                                                  float* __restrict__ sgate) {
  __shared__ uint32_t sel_key[4][kMaxK];
  __shared__ int sel_e[4][kMaxK];
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const uint16_t* lrow = logits + static_cast<int64_t>(t) * E;
  float z[EPL];
  uint32_t key[EPL];
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
    key[j] = e < E ? order_key(v) : 0u;   // 0 is below every valid key
    m = fmaxf(m, v);
  }
  m = wave_max(m);
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    if (j * kWave + lane < E) part += expf(z[j] - m);
  const float S = wave_sum(part);

  // Largest threshold with at least k keys >= threshold, built bit by bit from the top.
  uint32_t thr = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = thr | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) cnt += __popcll(__ballot(key[j] >= cand));
    if (cnt >= k) thr = cand;
  }
  int above = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) above += __popcll(__ballot(key[j] > thr));
  // Winners: every key above thr, then keys equal to thr in ascending expert index.
  int n_sel = 0, eq_seen = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const uint64_t eq = __ballot(key[j] == thr);
    const bool is_eq = key[j] == thr;
    const bool take = key[j] > thr || (is_eq && eq_seen + mask_rank(eq) < k - above);
    const uint64_t tk = __ballot(take);
    if (take) {
      const int pos = n_sel + mask_rank(tk);
      sel_key[wave][pos] = key[j];
      sel_e[wave][pos] = j * kWave + lane;
    }
    n_sel += __popcll(tk);
    eq_seen += __popcll(eq);
  }
  // sel_* rows are private to this wave, whose LDS accesses complete in program order.
  __builtin_amdgcn_wave_barrier();
  // Lane s < k owns winner s; its output slot is the number of winners ordered before it.
  float p = 0.f;
  int my_e = 0, slot = 0;
  if (lane < k) {
    const uint32_t mk = sel_key[wave][lane];
    my_e = sel_e[wave][lane];
    for (int i = 0; i < k; ++i) {
      const uint32_t ok = sel_key[wave][i];
      const int oe = sel_e[wave][i];
      slot += (ok > mk || (ok == mk && oe < my_e)) ? 1 : 0;
    }
    const uint32_t u = (mk & 0x80000000u) ? (mk & 0x7fffffffu) : ~mk;   // key -> z
    p = expf(__uint_as_float(u) - m) / S;
  }
  const float psum = wave_sum(p);
  if (lane < k) {
    const int64_t o = static_cast<int64_t>(t) * k + slot;
    topw[o] = static_cast<uint16_t>(f2bf(p / psum));
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
