// Weight-streaming grouped GEMMs for the bf16 MoE layer (gfx950, v_mfma_f32_16x16x32_bf16).
//
// Every GEMM of the layer has the form C[rows of W, tokens] = W[rows, K] . X[tokens, K]^T
// with both operands K-contiguous (the reference's nn.Linear / 3-D expert layouts,
// nanovllm/models/qwen3_5.py:765, :795-800, :912-914). A wave owns 16*RA weight rows and
// streams them from HBM once per pass over its group's tokens; the tokens (16 per MFMA
// column tile, TT tiles per pass) are read through L2. This is the decode-sized regime,
// where the layer is bound by streaming each hit expert's weights once.
//
// MFMA operand mapping. For v_mfma_f32_16x16x32_bf16 lane l = 16*q + r supplies row r of A
// and column r of B, 8 consecutive k each. K is walked in blocks of 128: in block kb lane
// (r, q) loads the 64 contiguous bytes k in [kb + 32q, kb + 32q + 32) of its weight row and
// of its token row, and MFMA c (c = 0..3) consumes the c-th 8-element chunk. A and B use the
// same (lane, chunk) -> k map, so the products pair correctly and each weight row is read
// as 256-byte contiguous segments. Accumulator lane (r, q) holds rows 4q..4q+3 of column r.
//
// Loads run kPD k-blocks ahead of the MFMAs. When K/128 is one of the unrolled sizes the
// whole K loop is unrolled so that the load of block i+kPD and the MFMAs of block i are
// statically scheduled; other sizes use a rolled loop with one block of lookahead.
#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

constexpr int kKBlock = 128;
#ifndef LBMOE_STREAM_PD
#define LBMOE_STREAM_PD 2
#endif
constexpr int kPD = LBMOE_STREAM_PD;   // k-blocks of loads in flight ahead of the MFMAs

template <int RA, int TT>
__device__ __forceinline__ void load_kblock(const uint16_t* const (&arow)[RA],
                                            const uint16_t* const (&brow)[TT], int k0,
                                            u32x4 (&a)[RA][4], u32x4 (&b)[TT][4]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      a[i][c] = ld16_stream(arow[i] + k0 + 8 * c);
#pragma unroll
  for (int j = 0; j < TT; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      b[j][c] = ld16(brow[j] + k0 + 8 * c);
}

template <int RA, int TT>
__device__ __forceinline__ void mma_kblock(const u32x4 (&a)[RA][4], const u32x4 (&b)[TT][4],
                                           f32x4 (&acc)[RA][TT]) {
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < RA; ++i)
#pragma unroll
      for (int j = 0; j < TT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[i][c]), as_bf16x8(b[j][c]),
                                                            acc[i][j], 0, 0, 0);
}

// acc[i][j] += W-tile i . X-tile j over NKB k-blocks (fully unrolled, kPD blocks in flight).
// arow/brow are this lane's row pointers, already offset by 32*q. Every pointer must be valid:
// loads are unconditional, so that the compiler can count the loads in flight exactly and keep
// the prefetch; a padding row (a token past the group, say) points at a real row and its
// output column is simply not stored.
template <int RA, int TT, int NKB>
__device__ __forceinline__ void stream_mma_fixed(const uint16_t* const (&arow)[RA],
                                                 const uint16_t* const (&brow)[TT],
                                                 f32x4 (&acc)[RA][TT]) {
  u32x4 a[NKB][RA][4], b[NKB][TT][4];
#pragma unroll
  for (int p = 0; p < kPD && p < NKB; ++p) load_kblock<RA, TT>(arow, brow, p * kKBlock, a[p], b[p]);
#pragma unroll
  for (int i = 0; i < NKB; ++i) {
    if (i + kPD < NKB) load_kblock<RA, TT>(arow, brow, (i + kPD) * kKBlock, a[i + kPD], b[i + kPD]);
    mma_kblock<RA, TT>(a[i], b[i], acc);
  }
}

// Rolled variant for any K (multiple of 128), one block of lookahead.
template <int RA, int TT>
__device__ __forceinline__ void stream_mma(const uint16_t* const (&arow)[RA],
                                           const uint16_t* const (&brow)[TT], int K,
                                           f32x4 (&acc)[RA][TT]) {
  u32x4 a[RA][4], b[TT][4], an[RA][4], bn[TT][4];
  load_kblock<RA, TT>(arow, brow, 0, a, b);
  for (int kb = 0; kb < K; kb += kKBlock) {
    if (kb + kKBlock < K) load_kblock<RA, TT>(arow, brow, kb + kKBlock, an, bn);
    mma_kblock<RA, TT>(a, b, acc);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int i = 0; i < RA; ++i) a[i][c] = an[i][c];
#pragma unroll
      for (int j = 0; j < TT; ++j) b[j][c] = bn[j][c];
    }
  }
}

// NKB = 0 selects the rolled loop over K.
template <int RA, int TT, int NKB>
__device__ __forceinline__ void stream_dot(const uint16_t* const (&arow)[RA],
                                           const uint16_t* const (&brow)[TT], int K,
                                           f32x4 (&acc)[RA][TT]) {
  if constexpr (NKB > 0) stream_mma_fixed<RA, TT, NKB>(arow, brow, acc);
  else stream_mma<RA, TT>(arow, brow, K, acc);
}

template <int RA, int TT>
__device__ __forceinline__ void zero_acc(f32x4 (&acc)[RA][TT]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// ---- wide loads + per-wave LDS transpose ---------------------------------------------------
// HBM streams best when each load instruction covers few rows with long contiguous runs. Here
// one instruction loads 4 rows x 256 contiguous bytes (16 lanes per row, 16 bytes each): lane l
// holds row 4u + l/16 (u = instruction), chunk l%16 of the row's 128-element k-block. The MFMA
// needs row r in lane r (mod 16), so each wave writes its k-block to a private LDS scratch and
// reads it back transposed. Chunk j of scratch row R sits at slot 16R + (j ^ (R & 15)), which
// keeps both the 16-lane row writes and the 16-row column reads free of bank conflicts.
// MFMA c of a k-block consumes chunks 4c..4c+3: lane (r, q) gets chunk 4c + q of row r, i.e.
// k = kb + 32c + 8q .. +8 for both operands.
template <int RA, int TT>
__device__ __forceinline__ void wide_load(const uint16_t* const (&ap)[RA][4],
                                          const uint16_t* const (&bp)[TT][4], int k0,
                                          u32x4 (&a)[RA][4], u32x4 (&b)[TT][4]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) a[i][u] = ld16_stream(ap[i][u] + k0);
#pragma unroll
  for (int j = 0; j < TT; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) b[j][u] = ld16(bp[j][u] + k0);
}

template <int RA, int TT>
__device__ __forceinline__ void wide_mma(u32x4* __restrict__ lds, const u32x4 (&a)[RA][4],
                                         const u32x4 (&b)[TT][4], f32x4 (&acc)[RA][TT]) {
  const int l = lane_id(), r = l & 15, q = l >> 4;
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) lds[(16 * i + 4 * u + q) * 16 + (r ^ (4 * u + q))] = a[i][u];
#pragma unroll
  for (int j = 0; j < TT; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) lds[(16 * (RA + j) + 4 * u + q) * 16 + (r ^ (4 * u + q))] = b[j][u];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int sl = (4 * c + q) ^ r;
    u32x4 fa[RA], fb[TT];
#pragma unroll
    for (int i = 0; i < RA; ++i) fa[i] = lds[(16 * i + r) * 16 + sl];
#pragma unroll
    for (int j = 0; j < TT; ++j) fb[j] = lds[(16 * (RA + j) + r) * 16 + sl];
#pragma unroll
    for (int i = 0; i < RA; ++i)
#pragma unroll
      for (int j = 0; j < TT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(fa[i]), as_bf16x8(fb[j]),
                                                            acc[i][j], 0, 0, 0);
  }
}

// acc += A . B^T over NKB k-blocks, kPD blocks of loads in flight (NKB = 0: rolled loop over K
// with one block of lookahead). ap/bp are this lane's row pointers, already offset by its
// 16-byte chunk; all must be valid (padding rows point at real rows, their outputs unused).
template <int RA, int TT, int NKB>
__device__ __forceinline__ void wide_dot(u32x4* __restrict__ lds, const uint16_t* const (&ap)[RA][4],
                                         const uint16_t* const (&bp)[TT][4], int K,
                                         f32x4 (&acc)[RA][TT]) {
  if constexpr (NKB > 0) {
    u32x4 a[NKB][RA][4], b[NKB][TT][4];
#pragma unroll
    for (int p = 0; p < kPD && p < NKB; ++p) wide_load<RA, TT>(ap, bp, p * kKBlock, a[p], b[p]);
#pragma unroll
    for (int i = 0; i < NKB; ++i) {
      if (i + kPD < NKB) wide_load<RA, TT>(ap, bp, (i + kPD) * kKBlock, a[i + kPD], b[i + kPD]);
      wide_mma<RA, TT>(lds, a[i], b[i], acc);
    }
  } else {
    u32x4 a[RA][4], b[TT][4], an[RA][4], bn[TT][4];
    wide_load<RA, TT>(ap, bp, 0, a, b);
    for (int kb = 0; kb < K; kb += kKBlock) {
      if (kb + kKBlock < K) wide_load<RA, TT>(ap, bp, kb + kKBlock, an, bn);
      wide_mma<RA, TT>(lds, a, b, acc);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int i = 0; i < RA; ++i) a[i][u] = an[i][u];
#pragma unroll
        for (int j = 0; j < TT; ++j) b[j][u] = bn[j][u];
      }
    }
  }
}

// Calls f.template operator()<NKB>() with NKB = K/128 when that size is unrolled, else 0.
template <typename F>
static hipError_t with_nkb(int K, F&& f) {
  switch (K / kKBlock) {
    case 1: return f.template operator()<1>();
    case 2: return f.template operator()<2>();
    case 3: return f.template operator()<3>();
    case 4: return f.template operator()<4>();
    case 6: return f.template operator()<6>();
    case 8: return f.template operator()<8>();
    case 16: return f.template operator()<16>();
    default: return f.template operator()<0>();
  }
}

// ---- residual add + RMSNorm ahead of the block (qwen3_5.py:998-1002, :39-55) ---------------
// h = bf16(residual + hidden) is the new residual; the block's input is
// x = bf16((h * (1 / sqrt(mean(h^2) + eps))) * (1 + w_norm)), in fp32 as Qwen3_5RMSNorm does.

// Elementwise h of 8 bf16 pairs; returns the sum of squares of the rounded values.
__device__ __forceinline__ float add_bf8(const u32x4& a, const u32x4& b, u32x4& h) {
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = round_bf(bf_lo(a[j]) + bf_lo(b[j]));
    const float hi = round_bf(bf_hi(a[j]) + bf_hi(b[j]));
    h[j] = pack_bf2(lo, hi);
    sq += lo * lo + hi * hi;
  }
  return sq;
}
__device__ __forceinline__ u32x4 norm_bf8(const u32x4& h, const u32x4& w, float rn) {
  u32x4 x;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    x[j] = pack_bf2((bf_lo(h[j]) * rn) * (1.0f + bf_lo(w[j])),
                    (bf_hi(h[j]) * rn) * (1.0f + bf_hi(w[j])));
  return x;
}

// One wave per token: h written to res_out, x to x_out.
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const uint16_t* __restrict__ hidden,
                                                          const uint16_t* __restrict__ residual,
                                                          const uint16_t* __restrict__ norm_w,
                                                          float eps, int T, int H,
                                                          uint16_t* __restrict__ x_out,
                                                          uint16_t* __restrict__ res_out) {
  const int lane = lane_id();
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int64_t row = static_cast<int64_t>(t) * H;
  float sq = 0.f;
  for (int k = 8 * lane; k < H; k += 8 * kWave) {
    u32x4 h;
    sq += add_bf8(ld16(residual + row + k), ld16(hidden + row + k), h);
    *reinterpret_cast<u32x4*>(res_out + row + k) = h;
  }
  const float rn = 1.0f / sqrtf(wave_sum(sq) / static_cast<float>(H) + eps);
  for (int k = 8 * lane; k < H; k += 8 * kWave) {
    u32x4 h;
    add_bf8(ld16(residual + row + k), ld16(hidden + row + k), h);
    *reinterpret_cast<u32x4*>(x_out + row + k) = norm_bf8(h, ld16(norm_w + k), rn);
  }
}

// ---- router logits: logits[t, e] = bf16(x[t] . Wg[e]) ----------------------------------
// Decode sizes. Workgroup = 8 waves on one 16-expert x 16-token tile, wave w taking k-blocks
// [nkb*w/8, nkb*(w+1)/8) of K (at most MAXB of them), so that every load of the wave is issued
// before the first MFMA; the eight partial sums are added in LDS in a fixed order and
// rounded once. NORM: x is not read but formed from the residual add and RMSNorm of the
// decoder layer (below): each wave computes h and x for its k-blocks of the 16 token rows,
// the waves' sums of squares meet in LDS, and the workgroups of expert tile 0 also store h
// and x. Both variants run the same MFMA chains, so their logits are identical.
constexpr int kRouterWaves = 8;
struct NormIn {
  const uint16_t* hidden;
  const uint16_t* residual;
  const uint16_t* weight;
  float eps;
  uint16_t* x_out;
  uint16_t* res_out;
};

template <bool NORM, int MAXB>
__global__ __launch_bounds__(64 * kRouterWaves) void router_logits_kernel(
    const uint16_t* __restrict__ x, NormIn nm, const uint16_t* __restrict__ wg, int T, int E,
    int H, uint16_t* __restrict__ logits) {
  __shared__ f32x4 part[kRouterWaves - 1][64];
  __shared__ float ss[kRouterWaves][16];
  const int lane = lane_id(), r = lane & 15, q = lane >> 4, w = threadIdx.x >> 6;
  const int e0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
  const int nkb = H / kKBlock;
  const int kb0 = (nkb * w) / kRouterWaves, nb = (nkb * (w + 1)) / kRouterWaves - kb0;
  const int t = t0 + r;
  const bool tv = t < T;
  // rows past T or E are loaded from the last real row (loads stay unconditional, so the
  // compiler keeps them all in flight) and their results are not stored
  const int64_t row = static_cast<int64_t>(min(t, T - 1)) * H;
  const uint16_t* wrow = wg + static_cast<int64_t>(min(e0 + r, E - 1)) * H;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto mfma_blocks = [&](const u32x4 (&a)[MAXB][4], const u32x4 (&b)[MAXB][4], int n) {
#pragma unroll
    for (int i = 0; i < MAXB; ++i) {
      if (i >= n) break;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[i][c]), as_bf16x8(b[i][c]), acc,
                                                      0, 0, 0);
    }
  };
  if constexpr (NORM) {
    // one pass (the host guarantees nb <= MAXB); every wave reaches the barrier, also one
    // without k-blocks
    u32x4 a[MAXB][4], b[MAXB][4], c2[MAXB][4], nwv[MAXB][4];
#pragma unroll
    for (int i = 0; i < MAXB; ++i) {
      if (i >= nb) break;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = (kb0 + i) * kKBlock + 32 * q + 8 * c;
        a[i][c] = ld16_stream(wrow + k);
        b[i][c] = ld16(nm.residual + row + k);
        c2[i][c] = ld16(nm.hidden + row + k);
        nwv[i][c] = ld16(nm.weight + k);
      }
    }
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < MAXB; ++i) {
      if (i >= nb) break;
#pragma unroll
      for (int c = 0; c < 4; ++c) sq += add_bf8(b[i][c], c2[i][c], b[i][c]);     // b := h
    }
    sq += __shfl_xor(sq, 16, kWave);
    sq += __shfl_xor(sq, 32, kWave);
    if (q == 0) ss[w][r] = sq;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int v = 0; v < kRouterWaves; ++v) tot += ss[v][r];
    const float rn = 1.0f / sqrtf(tot / static_cast<float>(H) + nm.eps);
    const bool store = blockIdx.x == 0 && tv;
#pragma unroll
    for (int i = 0; i < MAXB; ++i) {
      if (i >= nb) break;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = (kb0 + i) * kKBlock + 32 * q + 8 * c;
        if (store) *reinterpret_cast<u32x4*>(nm.res_out + row + k) = b[i][c];
        b[i][c] = norm_bf8(b[i][c], nwv[i][c], rn);                                // b := x
        if (store) *reinterpret_cast<u32x4*>(nm.x_out + row + k) = b[i][c];
      }
    }
    mfma_blocks(a, b, nb);
  } else {
    // MAXB k-blocks per pass, every operand of a pass loaded before its first MFMA
    for (int base = 0; base < nb; base += MAXB) {
      u32x4 a[MAXB][4], b[MAXB][4];
#pragma unroll
      for (int i = 0; i < MAXB; ++i) {
        if (base + i >= nb) break;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int k = (kb0 + base + i) * kKBlock + 32 * q + 8 * c;
          a[i][c] = ld16_stream(wrow + k);
          b[i][c] = ld16(x + row + k);
        }
      }
      mfma_blocks(a, b, nb - base);
    }
  }
  if (w > 0) part[w - 1][lane] = acc;
  __syncthreads();
  if (w != 0 || !tv) return;
  f32x4 sum = acc;
#pragma unroll
  for (int i = 0; i < kRouterWaves - 1; ++i) sum += part[i][lane];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int e = e0 + 4 * q + v;
    if (e < E) logits[static_cast<int64_t>(t) * E + e] = static_cast<uint16_t>(f2bf(sum[v]));
  }
}

// Per-wave k-blocks the decode router keeps in registers at once: up to 4 per pass; the fused
// norm needs all of a wave's blocks in one pass and fits 2 (H <= 2048) without spilling.
constexpr int kRouterPassBlocks = 4;
constexpr int kRouterNormBlocks = 2;

template <bool NORM>
static hipError_t launch_router_decode(const uint16_t* x, const NormIn& nm, const void* wg,
                                       int64_t T, int E, int H, void* logits, hipStream_t s) {
  const dim3 grid((E + 15) / 16, static_cast<unsigned>((T + 15) / 16));
  const int per_wave = (H / kKBlock + kRouterWaves - 1) / kRouterWaves;
  const auto* w = static_cast<const uint16_t*>(wg);
  auto* lg = static_cast<uint16_t*>(logits);
  const int Ti = static_cast<int>(T);
#define LBMOE_ROUTER(B) \
  router_logits_kernel<NORM, B><<<grid, 64 * kRouterWaves, 0, s>>>(x, nm, w, Ti, E, H, lg)
  if (per_wave <= 1) LBMOE_ROUTER(1);
  else if constexpr (NORM) LBMOE_ROUTER(kRouterNormBlocks);
  else if (per_wave <= 2) LBMOE_ROUTER(2);
  else LBMOE_ROUTER(kRouterPassBlocks);
#undef LBMOE_ROUTER
  return hipGetLastError();
}

// Token count from which the router logits run as an LDS-tiled MFMA GEMM.
constexpr int64_t kTiledRouterMinTokens = 1024;

hipError_t launch_router_logits(const void* x, const void* wg, int64_t T, int E, int H,
                                void* logits, hipStream_t s) {
  if (T >= kTiledRouterMinTokens && tiled_router_supported(E, H))
    return launch_router_logits_tiled(x, wg, T, E, H, logits, s);
  return launch_router_decode<false>(static_cast<const uint16_t*>(x), NormIn{}, wg, T, E, H,
                                     logits, s);
}

hipError_t launch_add_rmsnorm_router(const void* hidden, const void* residual, const void* norm_w,
                                     float eps, const void* wg, int64_t T, int E, int H,
                                     void* logits, void* x_out, void* res_out, hipStream_t s) {
  const NormIn nm{static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(residual),
                  static_cast<const uint16_t*>(norm_w), eps, static_cast<uint16_t*>(x_out),
                  static_cast<uint16_t*>(res_out)};
  const int per_wave = (H / kKBlock + kRouterWaves - 1) / kRouterWaves;
  if (T < kTiledRouterMinTokens && per_wave <= kRouterNormBlocks)
    return launch_router_decode<true>(nullptr, nm, wg, T, E, H, logits, s);
  add_rmsnorm_kernel<<<static_cast<unsigned>((T + 3) / 4), 256, 0, s>>>(
      nm.hidden, nm.residual, nm.weight, eps, static_cast<int>(T), H, nm.x_out, nm.res_out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_router_logits(x_out, wg, T, E, H, logits, s);
}

// Token tiles per pass from the expected tokens per routed expert (T*k/E): enough columns
// that a typical expert's weights stream once, few enough to keep occupancy.
static int pick_tt(const GroupWeights& gw, int64_t T, int k) {
  const double avg = gw.g0 < gw.E ? static_cast<double>(T) * k / gw.E : static_cast<double>(T);
  if (avg <= 12.0) return 1;
  if (avg <= 28.0) return 2;
  return 4;
}

// ---- gate_up + SiLU*mul ------------------------------------------------------------------
// Wave (channel block cb, group g): gate rows [16cb, 16cb+16) and the matching up rows of
// expert g; act[row, 16cb + c] = bf16(silu(gate) * up) (chunk(2,-1) + silu*mul of
// qwen3_5.py:835-836).
template <int TT, int NKB>
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
  __shared__ u32x4 lds[(2 + TT) * 256];
  // wide-load row pointers: instruction u covers rows 4u .. 4u+3 of each 16-row tile
  const uint16_t* ap[2][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ap[0][u] = wgt + static_cast<int64_t>(c0 + 4 * u + q) * H + 8 * r;
    ap[1][u] = wup + static_cast<int64_t>(c0 + 4 * u + q) * H + 8 * r;
  }
  for (int p0 = 0; p0 < n; p0 += 16 * TT) {
    const uint16_t* bp[TT][4];
#pragma unroll
    for (int j = 0; j < TT; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + 16 * j + 4 * u + q, n - 1);   // past n: a real row, not stored
        const int tok = shared ? p : perm_tok[row0 + p];
        bp[j][u] = x + static_cast<int64_t>(tok) * H + 8 * r;
      }
    f32x4 acc[2][TT];
    zero_acc(acc);
    wide_dot<2, TT, NKB>(lds, ap, bp, H, acc);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
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

template <int TT>
static hipError_t launch_gate_up_tt(const GroupWeights& gw, const void* x, const int32_t* counts,
                                    const int32_t* offsets, const int32_t* perm_tok, int64_t T,
                                    int act_ld, void* act, hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  const dim3 grid(Imax / 16, gw.groups);
  return with_nkb(gw.H, [&]<int NKB>() {
    gate_up_bf16_kernel<TT, NKB><<<grid, 64, 0, s>>>(gw, static_cast<const uint16_t*>(x), counts,
                                                     offsets, perm_tok, static_cast<int>(T),
                                                     act_ld, static_cast<uint16_t*>(act));
    return hipGetLastError();
  });
}

hipError_t launch_gate_up_bf16(const GroupWeights& gw, const void* x, const int32_t* counts,
                               const int32_t* offsets, const int32_t* perm_tok, int64_t T,
                               int k, int act_ld, void* act, hipStream_t s) {
  switch (pick_tt(gw, T, k)) {
    case 1: return launch_gate_up_tt<1>(gw, x, counts, offsets, perm_tok, T, act_ld, act, s);
    case 2: return launch_gate_up_tt<2>(gw, x, counts, offsets, perm_tok, T, act_ld, act, s);
    default: return launch_gate_up_tt<4>(gw, x, counts, offsets, perm_tok, T, act_ld, act, s);
  }
}

// ---- down projection ---------------------------------------------------------------------
// Wave (row block hb, group g): output columns [32hb, 32hb+32) of H for every token row of the
// group: out[row, h] = bf16(act[row, :Ig] . Wd_g[h, :Ig]) (qwen3_5.py:837, :868, :917).
template <int TT, int NKB>
__global__ __launch_bounds__(64) void down_bf16_kernel(GroupWeights gw,
                                                       const uint16_t* __restrict__ act,
                                                       int act_ld,
                                                       const int32_t* __restrict__ counts,
                                                       const int32_t* __restrict__ offsets,
                                                       int T, int width,
                                                       uint16_t* __restrict__ out) {
  const int g = gw.g0 + blockIdx.y;
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  if (Ig != width) return;          // groups of another width run in their own launch
  const int n = shared ? T : counts[g];
  if (n == 0) return;
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  const int H = gw.H;
  const int h0 = blockIdx.x * 32;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const uint16_t* wd = shared ? static_cast<const uint16_t*>(gw.sh_down)
                              : static_cast<const uint16_t*>(gw.down) +
                                    static_cast<int64_t>(g) * H * gw.I;
  __shared__ u32x4 lds[(2 + TT) * 256];
  const uint16_t* ap[2][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ap[0][u] = wd + static_cast<int64_t>(h0 + 4 * u + q) * Ig + 8 * r;
    ap[1][u] = wd + static_cast<int64_t>(h0 + 16 + 4 * u + q) * Ig + 8 * r;
  }
  for (int p0 = 0; p0 < n; p0 += 16 * TT) {
    const uint16_t* bp[TT][4];
#pragma unroll
    for (int j = 0; j < TT; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + 16 * j + 4 * u + q, n - 1);   // past n: a real row, not stored
        bp[j][u] = act + static_cast<int64_t>(row0 + p) * act_ld + 8 * r;
      }
    f32x4 acc[2][TT];
    zero_acc(acc);
    wide_dot<2, TT, NKB>(lds, ap, bp, Ig, acc);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
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

template <int TT>
static hipError_t launch_down_tt(const GroupWeights& gw, const void* act, int act_ld,
                                 const int32_t* counts, const int32_t* offsets, int64_t T,
                                 void* out, hipStream_t s) {
  const dim3 grid(gw.H / 32, gw.groups);
  auto go = [&](int K) {
    return with_nkb(K, [&]<int NKB>() {
      down_bf16_kernel<TT, NKB><<<grid, 64, 0, s>>>(gw, static_cast<const uint16_t*>(act), act_ld,
                                                    counts, offsets, static_cast<int>(T), K,
                                                    static_cast<uint16_t*>(out));
      return hipGetLastError();
    });
  };
  // Routed experts (width I) and the shared expert (width Is) each get the kernel unrolled
  // for their width; a group whose width differs from the launch's exits at once.
  const bool has_routed = gw.g0 < gw.E;
  const bool has_shared = gw.g0 + gw.groups > gw.E;
  hipError_t e = hipSuccess;
  if (has_routed) e = go(gw.I);
  if (e == hipSuccess && has_shared && (!has_routed || gw.Is != gw.I)) e = go(gw.Is);
  return e;
}

hipError_t launch_down_bf16(const GroupWeights& gw, const void* act, int act_ld,
                            const int32_t* counts, const int32_t* offsets, int64_t T, int k,
                            void* out, hipStream_t s) {
  switch (pick_tt(gw, T, k)) {
    case 1: return launch_down_tt<1>(gw, act, act_ld, counts, offsets, T, out, s);
    case 2: return launch_down_tt<2>(gw, act, act_ld, counts, offsets, T, out, s);
    default: return launch_down_tt<4>(gw, act, act_ld, counts, offsets, T, out, s);
  }
}

}  // namespace lbmoe
