// Split-K workgroups of the bf16 weight-streaming decode GEMMs (stream_gemm.hip): the plan and
// the cross-wave reduction. A workgroup of W waves owns 32 weight rows (two 16-row MFMA tiles)
// of one group; wave w streams its own k-blocks of those rows and the W partial sums are added
// in LDS, in wave order. A k-block is 256 bytes of a row, one wide load per 4 rows.
#pragma once
#include "common.hpp"

namespace lbmoe {

// Launch bounds and LDS are sized for kSplitMaxWaves waves; the plans use at most
// kSplitPlanWaves. (Sizing for 4 made the compiler trade loads in flight for occupancy and ran
// slower: gate_up at 256 tokens 155 vs 141 us.)
constexpr int kSplitMaxWaves = 8;
constexpr int kSplitPlanWaves = 4;

// LDS of a split-K workgroup, in 16-byte units: the waves' transpose slots, later reused for
// the partial sums [wave][tile i][token tile j][lane].
template <int TT>
constexpr int split_lds_u4() {
  return kSplitMaxWaves * 256 > kSplitMaxWaves * 2 * TT * 64 ? kSplitMaxWaves * 256
                                                               : kSplitMaxWaves * 2 * TT * 64;
}

// Writes this wave's partial sums over its transpose slots' LDS (after every wave is done
// with its slot) and makes them visible to the workgroup.
template <int TT>
__device__ __forceinline__ void split_publish(u32x4* lds, int wv, const f32x4 (&acc)[2][TT]) {
  __syncthreads();
  f32x4* part = reinterpret_cast<f32x4*>(lds);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) part[((wv * 2 + i) * TT + j) * 64 + lane_id()] = acc[i][j];
  __syncthreads();
}

// Sum over the W waves, in wave order, of accumulator (tile i, token tile j) of lane l.
template <int TT>
__device__ __forceinline__ f32x4 split_sum(const u32x4* lds, int W, int i, int j, int l) {
  const f32x4* part = reinterpret_cast<const f32x4*>(lds);
  f32x4 v = part[(i * TT + j) * 64 + l];
  for (int w = 1; w < W; ++w) v += part[((w * 2 + i) * TT + j) * 64 + l];
  return v;
}

// Waves and k-blocks per chunk for an item of nkb 256-byte k-blocks. Measured on the bf16
// decode shapes:
// - gate_up with one token tile loads two k-blocks per chunk, as long as the workgroup keeps at
//   least 3 waves; every other case loads one: gate_up with two token tiles runs 27% faster
//   on single-block chunks (two blocks' operands would not fit next to each other without
//   halving occupancy), and down at I=768 with 3 waves x two 1-block chunks beats 3 waves x
//   one 2-block chunk (67.5 vs 70 us at 128 tokens, 78.5 vs 85.6 at 256);
// - 4 waves per workgroup beat 8 (gate_up at 128 tokens 135.8 -> 127.5 us, E=512 494 -> 476 us
//   for the layer): each wave then walks two chunks, and four workgroups share a CU.
// W = the largest divisor of the chunk count up to 4, so every wave gets the same k-blocks.
struct SplitPlan {
  int waves, maxb;
};
inline SplitPlan split_plan(int nkb, int TT, bool down) {
  auto waves_for = [](int chunks) {
    int w = kSplitPlanWaves;
    while (chunks % w != 0) --w;
    return w;
  };
  const bool pairs = !down && TT == 1 && nkb % 2 == 0;
  if (pairs && waves_for(nkb / 2) >= 3) return {waves_for(nkb / 2), 2};
  return {waves_for(nkb), 1};
}

// Calls f.template operator()<TT, MAXB>() for the plan's MAXB (split_plan gives MAXB = 2 only
// for one token tile).
template <int TT, typename F>
inline hipError_t with_maxb(const SplitPlan& plan, F&& f) {
  if constexpr (TT == 1) {
    if (plan.maxb == 2) return f.template operator()<TT, 2>();
  }
  return f.template operator()<TT, 1>();
}

}  // namespace lbmoe
