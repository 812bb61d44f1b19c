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

// One workgroup per token. Per group of SLOTS slots, the token's (row, weight) pairs are read
// first, then every thread issues its row loads together before accumulating, so the loads
// overlap; the shared expert's row goes out with the first group's. SLOTS covers k for the
// usual widths (8 for k <= 8, 10 for k <= 10), so all of a token's rows are in flight at once:
// with groups of 8 at k = 10 the last two slots and the shared row took two more round trips
// (E=512 T=4096 combine 39.9 -> 36.9 us, T=128 7.4 -> 6.4 us in event-separated calls; fp8
// T=16384, bound by its 805 MB, unchanged). All loads are unconditional (indices past k or rows of
// dropped pairs read a real entry and are masked afterwards): a load under a condition would
// make the compiler wait for every earlier load at the join. The expert-output rows are read
// once and y is written once, both non-temporally, so neither stream displaces cached data
// (Qwen3-30B-A3B T=8192: 58.8 -> 50.4 us; fp8 E=512 T=16384: 168 -> 147 us).
template <int SLOTS, bool SHARED>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ rows,
                                                      const int32_t* __restrict__ inv,
                                                      const uint16_t* __restrict__ topw,
                                                      const float* __restrict__ sgate, int T,
                                                      int k, int H, int sh_row0,
                                                      uint16_t* __restrict__ y) {
  const int t = blockIdx.x;
  const int32_t* inv_t = inv + static_cast<int64_t>(t) * k;
  const uint16_t* w_t = topw + static_cast<int64_t>(t) * k;
  const uint16_t* sh_row = rows + static_cast<int64_t>(sh_row0 + t) * H;
  for (int c = threadIdx.x * 8; c < H; c += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    u32x4 osh;
    if constexpr (SHARED) osh = ld16_stream(sh_row + c);
    for (int s0 = 0; s0 < k; s0 += SLOTS) {
      int p[SLOTS];
      float w[SLOTS];
#pragma unroll
      for (int i = 0; i < SLOTS; ++i) {
        const int s = min(s0 + i, k - 1);
        const bool in = s0 + i < k;
        p[i] = in ? inv_t[s] : -1;
        w[i] = bf2f(w_t[s]);
      }
      u32x4 o[SLOTS];
#pragma unroll
      for (int i = 0; i < SLOTS; ++i)
        o[i] = ld16_stream(rows + static_cast<int64_t>(max(p[i], 0)) * H + c);
#pragma unroll
      for (int i = 0; i < SLOTS; ++i) {
        const bool use = p[i] >= 0;        // dropped pairs and slots past k add nothing
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += use ? w[i] * bf_lo(o[i][q]) : 0.f;
          acc[2 * q + 1] += use ? w[i] * bf_hi(o[i][q]) : 0.f;
        }
      }
    }
    if constexpr (SHARED) {
      const float g = sgate[t];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += g * bf_lo(osh[q]);
        acc[2 * q + 1] += g * bf_hi(osh[q]);
      }
    }
    u32x4 pk;
#pragma unroll
    for (int q = 0; q < 4; ++q) pk[q] = pack_bf2(acc[2 * q], acc[2 * q + 1]);
    __builtin_nontemporal_store(pk, reinterpret_cast<u32x4*>(y + static_cast<int64_t>(t) * H + c));
  }
}

// ---- down projection + combine for the smallest batches -------------------------------------
// At T <= kFusedDownTokens the down GEMM's rows are so few that its launch, and the combine's
// after it, cost more than their memory traffic: one launch does both. Workgroup = kFusedCols
// output columns h0 .. h0+7 for every token; wave w takes entries j = w, w + 8, ... (entry
// t*k + s: token t's slot s, routed to expert idx[j], its act row inv[j]; entries T*k + t: the
// shared expert's row of token t) and computes out[j, h0 + r] = act[row] . Wd_e[h0 + r] for
// its 8 rows: lane (r, u) holds chunks u, u + 8, ... (16 bytes each) of weight row r and of the
// act row, so a load instruction reads 8 rows x 128 contiguous bytes, all of an entry's loads
// are in flight together, and the 8 lanes of a row meet in a butterfly sum. Each product is
// rounded to bf16 as the down GEMM stores it, and the combine then runs from LDS exactly as
// combine_kernel does (fp32 in slot order, then the gated shared term, one bf16 rounding).
// MAXC: chunks per lane for the widest expert (I or Is = 64 * MAXC).
constexpr int kFusedWaves = 8;
template <int MAXC>
__global__ __launch_bounds__(64 * kFusedWaves) void down_combine_small_kernel(
    GroupWeights gw, const uint16_t* __restrict__ act, int act_ld, const int32_t* __restrict__ idx,
    const int32_t* __restrict__ inv, const uint16_t* __restrict__ topw,
    const float* __restrict__ sgate, int T, int k, uint16_t* __restrict__ y) {
  __shared__ float s_out[kFusedDownEntries][kFusedCols];
  const int H = gw.H, h0 = blockIdx.x * kFusedCols;
  const int lane = lane_id(), r = lane >> 3, u = lane & 7;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int V = T * k, nent = V + (sgate != nullptr ? T : 0);
  for (int j = wv; j < nent; j += kFusedWaves) {           // the same for the whole wave
    const bool sh = j >= V;
    const int Ig = sh ? gw.Is : gw.I;
    // a pair whose expert id was out of range (inv < 0) contributes nothing; its loads read
    // expert 0's weights and act row 0
    const int iv = sh ? 0 : inv[j];
    const bool drop = iv < 0;
    const int row = sh ? gw.sh_row0 + (j - V) : (drop ? 0 : iv);
    const uint16_t* wbase = sh ? static_cast<const uint16_t*>(gw.sh_down)
                               : static_cast<const uint16_t*>(gw.down) +
                                     static_cast<int64_t>(drop ? 0 : idx[j]) * H * gw.I;
    const uint16_t* wrow = wbase + static_cast<int64_t>(h0 + r) * Ig;
    const uint16_t* arow = act + static_cast<int64_t>(row) * act_ld;
    const int nch = Ig / 8;
    // unconditional loads (chunks past the row re-read its last chunk and are not added)
    u32x4 wq[MAXC], aq[MAXC];
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int c = min(u + 8 * i, nch - 1);
      wq[i] = ld16_stream(wrow + 8 * c);
      aq[i] = ld16(arow + 8 * c);
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      if (u + 8 * i >= nch) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc += bf_lo(wq[i][q]) * bf_lo(aq[i][q]);
        acc += bf_hi(wq[i][q]) * bf_hi(aq[i][q]);
      }
    }
    acc += __shfl_xor(acc, 1, kWave);
    acc += __shfl_xor(acc, 2, kWave);
    acc += __shfl_xor(acc, 4, kWave);
    if (u == 0) s_out[j][r] = drop ? 0.f : round_bf(acc);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * kFusedCols; i += blockDim.x) {
    const int t = i / kFusedCols, col = i - t * kFusedCols;
    float a = 0.f;
    for (int s = 0; s < k; ++s) a += bf2f(topw[t * k + s]) * s_out[t * k + s][col];
    if (sgate != nullptr) a += sgate[t] * s_out[V + t][col];
    y[static_cast<int64_t>(t) * H + h0 + col] = static_cast<uint16_t>(f2bf(a));
  }
}

bool down_combine_small_supported(const GroupWeights& gw, int64_t T, int k) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  return T >= 1 && T <= kFusedDownTokens && T * k + T <= kFusedDownEntries &&
         gw.H % kFusedCols == 0 && Imax <= 64 * 16 && gw.I % 64 == 0 && gw.Is % 64 == 0;
}

hipError_t launch_down_combine_small(const GroupWeights& gw, const void* act, int act_ld,
                                     const int32_t* idx, const int32_t* inv, const void* topw,
                                     const float* sgate, int64_t T, int k, bool shared, void* y,
                                     hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  const dim3 grid(gw.H / kFusedCols);
  const auto* a = static_cast<const uint16_t*>(act);
  const auto* tw = static_cast<const uint16_t*>(topw);
  const float* g = shared ? sgate : nullptr;
  auto* yy = static_cast<uint16_t*>(y);
  const int Ti = static_cast<int>(T);
  if (Imax <= 512)
    down_combine_small_kernel<8><<<grid, 64 * kFusedWaves, 0, s>>>(gw, a, act_ld, idx, inv, tw, g, Ti, k, yy);
  else if (Imax <= 768)
    down_combine_small_kernel<12><<<grid, 64 * kFusedWaves, 0, s>>>(gw, a, act_ld, idx, inv, tw, g, Ti, k, yy);
  else
    down_combine_small_kernel<16><<<grid, 64 * kFusedWaves, 0, s>>>(gw, a, act_ld, idx, inv, tw, g, Ti, k, yy);
  return hipGetLastError();
}

hipError_t launch_combine(const void* out_rows, const int32_t* inv, const void* topw,
                          const float* sgate, int64_t T, int k, int H, bool shared, void* y,
                          hipStream_t s) {
#define LBMOE_COMBINE(SLOTS, SH)                                                              \
  combine_kernel<SLOTS, SH><<<static_cast<unsigned>(T), 256, 0, s>>>(                         \
      static_cast<const uint16_t*>(out_rows), inv, static_cast<const uint16_t*>(topw), sgate,  \
      static_cast<int>(T), k, H, static_cast<int>(T) * k, static_cast<uint16_t*>(y))
  if (shared) {
    if (k <= 8) LBMOE_COMBINE(8, true);
    else if (k <= 10) LBMOE_COMBINE(10, true);
    else LBMOE_COMBINE(8, true);
  } else {
    if (k <= 8) LBMOE_COMBINE(8, false);
    else if (k <= 10) LBMOE_COMBINE(10, false);
    else LBMOE_COMBINE(8, false);
  }
#undef LBMOE_COMBINE
  return hipGetLastError();
}

}  // namespace lbmoe
