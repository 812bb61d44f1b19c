// Weight-streaming grouped GEMMs for the bf16 MoE layer (gfx950, v_mfma_f32_16x16x32_bf16).
//
// Every GEMM of the layer has the form C[rows of W, tokens] = W[rows, K] . X[tokens, K]^T
// with both operands K-contiguous (the reference's nn.Linear / 3-D expert layouts,
// nanovllm/models/qwen3_5.py:765, :795-800, :912-914). A wave owns 16*RA weight rows and
// streams them from HBM exactly once per pass over its group's tokens; the tokens (16 per
// MFMA column tile, TT tiles per pass) are read through L2.
//
// MFMA operand mapping. For v_mfma_f32_16x16x32_bf16 lane l = 16*q + r supplies row r of A
// and column r of B, 8 consecutive k each. K is walked in blocks of 128: in block kb lane
// (r, q) loads the 64 contiguous bytes k in [kb + 32q, kb + 32q + 32) of its weight row and
// of its token row, and MFMA c (c = 0..3) consumes the c-th 8-element chunk. A and B use the
// same (lane, chunk) -> k map, so the products pair correctly and each weight row is read
// as 256-byte contiguous segments. Accumulator lane (r, q) holds rows 4q..4q+3 of column r.
#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

constexpr int kKBlock = 128;

template <int RA, int TT>
__device__ __forceinline__ void load_kblock(const uint16_t* const (&arow)[RA],
                                            const uint16_t* const (&brow)[TT], int k0,
                                            u32x4 (&a)[RA][4], u32x4 (&b)[TT][4]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      a[i][c] = arow[i] ? ld16_stream(arow[i] + k0 + 8 * c) : u32x4{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < TT; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      b[j][c] = brow[j] ? ld16(brow[j] + k0 + 8 * c) : u32x4{0, 0, 0, 0};
}

// acc[i][j] += W-tile i . X-tile j over K (K a multiple of 128). arow/brow are this lane's
// row pointers (nullptr = zero row), already offset by 32*q.
template <int RA, int TT>
__device__ __forceinline__ void stream_mma(const uint16_t* const (&arow)[RA],
                                           const uint16_t* const (&brow)[TT], int K,
                                           f32x4 (&acc)[RA][TT]) {
  u32x4 a[RA][4], b[TT][4], an[RA][4], bn[TT][4];
  load_kblock<RA, TT>(arow, brow, 0, a, b);
  for (int kb = 0; kb < K; kb += kKBlock) {
    if (kb + kKBlock < K) load_kblock<RA, TT>(arow, brow, kb + kKBlock, an, bn);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < RA; ++i)
#pragma unroll
        for (int j = 0; j < TT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[i][c]),
                                                              as_bf16x8(b[j][c]), acc[i][j],
                                                              0, 0, 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int i = 0; i < RA; ++i) a[i][c] = an[i][c];
#pragma unroll
      for (int j = 0; j < TT; ++j) b[j][c] = bn[j][c];
    }
  }
}

template <int RA, int TT>
__device__ __forceinline__ void zero_acc(f32x4 (&acc)[RA][TT]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// ---- router logits: logits[t, e] = bf16(x[t] . Wg[e]) ----------------------------------
constexpr int kRouterTT = 2;

__global__ __launch_bounds__(64) void router_logits_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ wg,
                                                           int T, int E, int H,
                                                           uint16_t* __restrict__ logits) {
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const int e0 = blockIdx.x * 16;
  const int t0 = blockIdx.y * 16 * kRouterTT;
  const uint16_t* arow[1] = {e0 + r < E ? wg + static_cast<int64_t>(e0 + r) * H + 32 * q
                                        : nullptr};
  const uint16_t* brow[kRouterTT];
#pragma unroll
  for (int j = 0; j < kRouterTT; ++j) {
    const int t = t0 + 16 * j + r;
    brow[j] = t < T ? x + static_cast<int64_t>(t) * H + 32 * q : nullptr;
  }
  f32x4 acc[1][kRouterTT];
  zero_acc(acc);
  stream_mma<1, kRouterTT>(arow, brow, H, acc);
#pragma unroll
  for (int j = 0; j < kRouterTT; ++j) {
    const int t = t0 + 16 * j + r;
    if (t >= T) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int e = e0 + 4 * q + v;
      if (e < E) logits[static_cast<int64_t>(t) * E + e] = static_cast<uint16_t>(f2bf(acc[0][j][v]));
    }
  }
}

hipError_t launch_router_logits(const void* x, const void* wg, int64_t T, int E, int H,
                                void* logits, hipStream_t s) {
  const dim3 grid((E + 15) / 16, static_cast<unsigned>((T + 16 * kRouterTT - 1) / (16 * kRouterTT)));
  router_logits_kernel<<<grid, 64, 0, s>>>(static_cast<const uint16_t*>(x),
                                           static_cast<const uint16_t*>(wg),
                                           static_cast<int>(T), E, H,
                                           static_cast<uint16_t*>(logits));
  return hipGetLastError();
}

// ---- gate_up + SiLU*mul ------------------------------------------------------------------
// Wave (channel block cb, group g): gate rows [16cb, 16cb+16) and the matching up rows of
// expert g; act[row, 16cb + c] = bf16(silu(gate) * up) (chunk(2,-1) + silu*mul of
// qwen3_5.py:835-836).
constexpr int kGateUpTT = 2;

__global__ __launch_bounds__(64) void gate_up_bf16_kernel(GroupWeights gw,
                                                          const uint16_t* __restrict__ x,
                                                          const int32_t* __restrict__ counts,
                                                          const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ perm_tok,
                                                          int T, int act_ld,
                                                          uint16_t* __restrict__ act) {
  const int g = gw.g0 + blockIdx.y;
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int c0 = blockIdx.x * 16;
  if (c0 >= Ig) return;
  const int n = shared ? T : counts[g];
  if (n == 0) return;
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  const int H = gw.H;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const uint16_t* wgt;
  const uint16_t* wup;
  if (shared) {
    wgt = static_cast<const uint16_t*>(gw.sh_gate);
    wup = static_cast<const uint16_t*>(gw.sh_up);
  } else {
    wgt = static_cast<const uint16_t*>(gw.gate_up) + static_cast<int64_t>(g) * 2 * gw.I * H;
    wup = wgt + static_cast<int64_t>(gw.I) * H;
  }
  const uint16_t* arow[2] = {wgt + static_cast<int64_t>(c0 + r) * H + 32 * q,
                             wup + static_cast<int64_t>(c0 + r) * H + 32 * q};
  for (int p0 = 0; p0 < n; p0 += 16 * kGateUpTT) {
    const uint16_t* brow[kGateUpTT];
#pragma unroll
    for (int j = 0; j < kGateUpTT; ++j) {
      const int p = p0 + 16 * j + r;
      const int tok = p < n ? (shared ? p : perm_tok[row0 + p]) : -1;
      brow[j] = tok >= 0 ? x + static_cast<int64_t>(tok) * H + 32 * q : nullptr;
    }
    f32x4 acc[2][kGateUpTT];
    zero_acc(acc);
    stream_mma<2, kGateUpTT>(arow, brow, H, acc);
#pragma unroll
    for (int j = 0; j < kGateUpTT; ++j) {
      const int p = p0 + 16 * j + r;
      if (p >= n) continue;
      float a[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) a[v] = silu(acc[0][j][v]) * acc[1][j][v];
      u32x2 pk = {pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
      *reinterpret_cast<u32x2*>(act + static_cast<int64_t>(row0 + p) * act_ld + c0 + 4 * q) = pk;
    }
  }
}


hipError_t launch_gate_up_bf16(const GroupWeights& gw, const void* x, const int32_t* counts,
                               const int32_t* offsets, const int32_t* perm_tok, int64_t T,
                               int act_ld, void* act, hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  const dim3 grid(Imax / 16, gw.groups);
  gate_up_bf16_kernel<<<grid, 64, 0, s>>>(gw, static_cast<const uint16_t*>(x), counts, offsets,
                                          perm_tok, static_cast<int>(T), act_ld,
                                          static_cast<uint16_t*>(act));
  return hipGetLastError();
}

// ---- down projection ---------------------------------------------------------------------
// Wave (row block hb, group g): output columns [32hb, 32hb+32) of H for every token row of the
// group: out[row, h] = bf16(act[row, :Ig] . Wd_g[h, :Ig]) (qwen3_5.py:837, :868, :917).
constexpr int kDownTT = 2;

__global__ __launch_bounds__(64) void down_bf16_kernel(GroupWeights gw,
                                                       const uint16_t* __restrict__ act,
                                                       int act_ld,
                                                       const int32_t* __restrict__ counts,
                                                       const int32_t* __restrict__ offsets,
                                                       int T, uint16_t* __restrict__ out) {
  const int g = gw.g0 + blockIdx.y;
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int n = shared ? T : counts[g];
  if (n == 0) return;
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  const int H = gw.H;
  const int h0 = blockIdx.x * 32;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const uint16_t* wd = shared ? static_cast<const uint16_t*>(gw.sh_down)
                              : static_cast<const uint16_t*>(gw.down) +
                                    static_cast<int64_t>(g) * H * gw.I;
  const uint16_t* arow[2] = {wd + static_cast<int64_t>(h0 + r) * Ig + 32 * q,
                             wd + static_cast<int64_t>(h0 + 16 + r) * Ig + 32 * q};
  for (int p0 = 0; p0 < n; p0 += 16 * kDownTT) {
    const uint16_t* brow[kDownTT];
#pragma unroll
    for (int j = 0; j < kDownTT; ++j) {
      const int p = p0 + 16 * j + r;
      brow[j] = p < n ? act + static_cast<int64_t>(row0 + p) * act_ld + 32 * q : nullptr;
    }
    f32x4 acc[2][kDownTT];
    zero_acc(acc);
    stream_mma<2, kDownTT>(arow, brow, Ig, acc);
#pragma unroll
    for (int j = 0; j < kDownTT; ++j) {
      const int p = p0 + 16 * j + r;
      if (p >= n) continue;
      uint16_t* orow = out + static_cast<int64_t>(row0 + p) * H + h0 + 4 * q;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        u32x2 pk = {pack_bf2(acc[i][j][0], acc[i][j][1]), pack_bf2(acc[i][j][2], acc[i][j][3])};
        *reinterpret_cast<u32x2*>(orow + 16 * i) = pk;
      }
    }
  }
}

hipError_t launch_down_bf16(const GroupWeights& gw, const void* act, int act_ld,
                            const int32_t* counts, const int32_t* offsets, int64_t T,
                            void* out, hipStream_t s) {
  const dim3 grid(gw.H / 32, gw.groups);
  down_bf16_kernel<<<grid, 64, 0, s>>>(gw, static_cast<const uint16_t*>(act), act_ld, counts,
                                       offsets, static_cast<int>(T),
                                       static_cast<uint16_t*>(out));
  return hipGetLastError();
}

}  // namespace lbmoe
