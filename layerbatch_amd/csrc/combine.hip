// Top-k weighted unpermute-combine (deterministic, no atomics).
//
// y[t] = bf16( sum_s w[t,s] * out[inv[t,s]]  +  gate[t] * out[sh_row0 + t] )
// The routed sum is the weighted slot sum of the reference (qwen3_5.py:871-872, dense path;
// the sparse path's index_add_, :838-839, adds the same terms), the second term is the gated
// shared expert (qwen3_5.py:903-904). Accumulation is fp32 in slot order 0..k-1, then the
// shared term, with one rounding to bf16 at the end. Pairs with inv < 0 (expert id out of
// range) contribute nothing.
#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

// One workgroup per token. Per group of kCombineSlots slots, the token's (row, weight) pairs
// are read first, then every thread issues its row loads together before accumulating, so the
// loads overlap. All loads are unconditional (indices past k or rows of dropped pairs read a
// real entry and are masked afterwards): a load under a condition would make the compiler
// wait for every earlier load at the join.
constexpr int kCombineSlots = 8;   // slots whose row loads are in flight together

__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ rows,
                                                      const int32_t* __restrict__ inv,
                                                      const uint16_t* __restrict__ topw,
                                                      const float* __restrict__ sgate, int T,
                                                      int k, int H, int sh_row0,
                                                      uint16_t* __restrict__ y) {
  const int t = blockIdx.x;
  const int32_t* inv_t = inv + static_cast<int64_t>(t) * k;
  const uint16_t* w_t = topw + static_cast<int64_t>(t) * k;
  for (int c = threadIdx.x * 8; c < H; c += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < k; s0 += kCombineSlots) {
      int p[kCombineSlots];
      float w[kCombineSlots];
#pragma unroll
      for (int i = 0; i < kCombineSlots; ++i) {
        const int s = min(s0 + i, k - 1);
        const bool in = s0 + i < k;
        p[i] = in ? inv_t[s] : -1;
        w[i] = bf2f(w_t[s]);
      }
      u32x4 o[kCombineSlots];
#pragma unroll
      for (int i = 0; i < kCombineSlots; ++i)
        o[i] = ld16(rows + static_cast<int64_t>(max(p[i], 0)) * H + c);
#pragma unroll
      for (int i = 0; i < kCombineSlots; ++i) {
        const bool use = p[i] >= 0;        // dropped pairs and slots past k add nothing
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += use ? w[i] * bf_lo(o[i][q]) : 0.f;
          acc[2 * q + 1] += use ? w[i] * bf_hi(o[i][q]) : 0.f;
        }
      }
    }
    if (sgate != nullptr) {
      const float g = sgate[t];
      const u32x4 o = ld16(rows + static_cast<int64_t>(sh_row0 + t) * H + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += g * bf_lo(o[q]);
        acc[2 * q + 1] += g * bf_hi(o[q]);
      }
    }
    u32x4 pk;
#pragma unroll
    for (int q = 0; q < 4; ++q) pk[q] = pack_bf2(acc[2 * q], acc[2 * q + 1]);
    *reinterpret_cast<u32x4*>(y + static_cast<int64_t>(t) * H + c) = pk;
  }
}

hipError_t launch_combine(const void* out_rows, const int32_t* inv, const void* topw,
                          const float* sgate, int64_t T, int k, int H, bool shared, void* y,
                          hipStream_t s) {
  combine_kernel<<<static_cast<unsigned>(T), 256, 0, s>>>(
      static_cast<const uint16_t*>(out_rows), inv, static_cast<const uint16_t*>(topw),
      shared ? sgate : nullptr, static_cast<int>(T), k, H, static_cast<int>(T) * k,
      static_cast<uint16_t*>(y));
  return hipGetLastError();
}

}  // namespace lbmoe
