// Weight-streaming grouped GEMMs for the bf16 MoE layer (gfx950, v_mfma_f32_16x16x32_bf16).
//
// Every GEMM of the layer has the form C[rows of W, tokens] = W[rows, K] . X[tokens, K]^T
// with both operands K-contiguous (the reference's nn.Linear / 3-D expert layouts,
// nanovllm/models/qwen3_5.py:765, :795-800, :912-914). This is the decode-sized regime, where
// the layer is bound by streaming each hit expert's weights from HBM once.
//
// Split-K workgroups. A workgroup of W waves owns one item: 32 weight rows (two 16-row MFMA
// tiles) of one group against all of the group's tokens (16 per MFMA column tile, TT tiles per
// pass). Wave w streams k-blocks [w*per, (w+1)*per) of the 32 rows, per = K/128/W, issuing all
// loads of MAXB k-blocks before its first MFMA, so the item's 32 x K weight block is in flight
// at once, as one burst of neighbouring addresses. HBM streams such bursts markedly faster
// than one long per-wave stream per row block (a bandwidth probe: 6.5-6.9 TB/s against
// 5.7-6.2 TB/s over 0.75-1.5 GB). The W partial sums meet in LDS and are added in wave order,
// a fixed order, so results do not depend on timing.
//
// Wide loads. One load instruction covers 4 rows x 256 contiguous bytes (16 lanes per row,
// 16 bytes each): lane l holds row 4u + l/16 (u = instruction), chunk l%16 of the row's
// 128-element k-block. v_mfma_f32_16x16x32_bf16 wants row r in lane r (mod 16), so each 16 x
// 128 tile passes through a private 4 KB LDS slot of the wave: chunk j of row R sits at slot
// 16R + (j ^ (R & 15)), free of bank conflicts for both the 16-lane row writes and the 16-row
// column reads. MFMA c of a k-block consumes chunks 4c..4c+3: lane (r, q) gets chunk 4c + q of
// row r, k = kb + 32c + 8q .. +8, for both operands, so the products pair correctly. A wave's
// LDS operations execute in issue order, so the slot is reused tile after tile without waits.
// Accumulator lane (r, q) holds rows 4q..4q+3 of column r.
#include "common.hpp"
#include "internal.hpp"
#include "route_token.hpp"
#include "split_k.hpp"

namespace lbmoe {

constexpr int kKBlock = 128;

// Loads k-block kb of both weight tiles and of the TT token tiles. abase[i] is tile i's
// wave-uniform base, astep the uniform byte step between load instructions (4 rows) and aoff
// this lane's 32-bit byte offset, so the weight loads take the scalar-base form. Every pointer must be valid: padding token rows point at real rows and
// their outputs are not stored, so the loads stay unconditional and the compiler can count
// those in flight exactly.
template <int TT>
__device__ __forceinline__ void split_load(const char* const (&abase)[2], int astep, uint32_t aoff,
                                           const uint16_t* const (&bp)[TT][4], int kb,
                                           u32x4 (&a)[2][4], u32x4 (&b)[TT][4]) {
  const int kbyte = kb * kKBlock * 2;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) a[i][u] = ld16_stream(abase[i] + (kbyte + u * astep) + aoff);
#pragma unroll
  for (int j = 0; j < TT; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) b[j][u] = ld16(bp[j][u] + kb * kKBlock);
}

// acc += A . B^T over one k-block, each tile transposed through the wave's LDS slot. The
// token tiles go first and each weight tile's MFMAs follow its transpose, so that few
// fragments are live next to the loads still in flight.
template <int TT>
__device__ __forceinline__ void split_mma(u32x4* __restrict__ slot, const u32x4 (&a)[2][4],
                                          const u32x4 (&b)[TT][4], f32x4 (&acc)[2][TT]) {
  const int l = lane_id(), r = l & 15, q = l >> 4;
  auto transpose = [&](const u32x4 (&t)[4], u32x4 (&f)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) slot[(4 * u + q) * 16 + (r ^ (4 * u + q))] = t[u];
#pragma unroll
    for (int c = 0; c < 4; ++c) f[c] = slot[r * 16 + ((4 * c + q) ^ r)];
  };
  u32x4 fb[TT][4];
#pragma unroll
  for (int j = 0; j < TT; ++j) transpose(b[j], fb[j]);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    u32x4 fa[4];
    transpose(a[i], fa);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int j = 0; j < TT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(fa[c]), as_bf16x8(fb[j][c]),
                                                            acc[i][j], 0, 0, 0);
  }
}

// This wave's share of the item: acc = sum over k-blocks [kb0, kb0 + per) in chunks of MAXB.
template <int TT, int MAXB>
__device__ __forceinline__ void split_dot(u32x4* __restrict__ slot, const char* const (&abase)[2],
                                          int astep, uint32_t aoff,
                                          const uint16_t* const (&bp)[TT][4], int kb0, int per,
                                          f32x4 (&acc)[2][TT]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kb = kb0; kb < kb0 + per; kb += MAXB) {
    u32x4 a[MAXB][2][4], b[MAXB][TT][4];
#pragma unroll
    for (int m = 0; m < MAXB; ++m) split_load<TT>(abase, astep, aoff, bp, kb + m, a[m], b[m]);
#pragma unroll
    for (int m = 0; m < MAXB; ++m) split_mma<TT>(slot, a[m], b[m], acc);
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
// rounded once. MFMA c of a k-block takes its 32 k in the operand layout straight from
// memory: lane (r, q) loads k = 32c + 8q .. +8 of row r, so the four lanes of a row cover one
// 64-byte segment and a load instruction touches 16 segments. (With k = 32q + 8c every
// instruction touched 64 segments, 16 bytes of each, and the texture-address unit, at about
// one segment per cycle, bounded the kernel.) NORM: x is not read but formed from the residual add and RMSNorm of the
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
        const int k = (kb0 + i) * kKBlock + 32 * c + 8 * q;
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
        const int k = (kb0 + i) * kKBlock + 32 * c + 8 * q;
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
          const int k = (kb0 + base + i) * kKBlock + 32 * c + 8 * q;
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

bool router_is_tiled(int64_t T, int E, int H) {
  // the tiled router's buffer copies address x and the gate weight with byte offsets < 2^31
  return T >= kTiledRouterMinTokens && tiled_router_supported(E, H) &&
         T * H * 2 < (int64_t{1} << 31);
}

hipError_t launch_router_logits(const void* x, const void* wg, int64_t T, int E, int H,
                                void* logits, hipStream_t s) {
  if (router_is_tiled(T, E, H))
    return launch_router_logits_tiled(x, wg, T, E, H, logits, s);
  return launch_router_decode<false>(static_cast<const uint16_t*>(x), NormIn{}, wg, T, E, H,
                                     logits, s);
}

// Token count up to which the norm runs inside the router. Every expert tile's workgroup
// recomputes its tokens' norm and cannot start its MFMAs before the whole row is summed, so
// the fused kernel loses to add_rmsnorm_kernel + the plain router as T grows (Qwen3-30B-A3B
// layer, back-to-back calls: T=1 41.5 vs 42.7 us, T=32 185.4 vs 184.4, T=128 227.0 vs 224.6,
// T=512 431 vs 422).
constexpr int64_t kNormFusedMaxTokens = 16;

hipError_t launch_add_rmsnorm_router(const void* hidden, const void* residual, const void* norm_w,
                                     float eps, const void* wg, int64_t T, int E, int H,
                                     void* logits, void* x_out, void* res_out, hipStream_t s) {
  const NormIn nm{static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(residual),
                  static_cast<const uint16_t*>(norm_w), eps, static_cast<uint16_t*>(x_out),
                  static_cast<uint16_t*>(res_out)};
  const int per_wave = (H / kKBlock + kRouterWaves - 1) / kRouterWaves;
  if (T <= kNormFusedMaxTokens && per_wave <= kRouterNormBlocks)
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
  if (avg <= 8.0) return 1;   // above, many groups would need two passes of 16 tokens
  if (avg <= 28.0) return 2;
  return 4;
}

// ---- gate_up + SiLU*mul ------------------------------------------------------------------
// Workgroup (channel block cb, group g): gate rows [16cb, 16cb+16) and the matching up rows of
// expert g; act[row, 16cb + c] = bf16(silu(gate) * up) (chunk(2,-1) + silu*mul of
// qwen3_5.py:835-836). Group g has n rows from row0 on; toks[p] is the token of its row p
// (not read for the shared expert, whose row p is token p).
template <int TT, int MAXB>
__device__ __forceinline__ void gate_up_group(const GroupWeights& gw, const uint16_t* __restrict__ x,
                                              int g, int n, int row0, const int32_t* toks,
                                              int slice, int nslices, int act_ld,
                                              uint16_t* __restrict__ act, u32x4* lds) {
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int c0 = blockIdx.x * 16;
  if (c0 >= Ig || n == 0) return;
  const int H = gw.H;
  const int W = blockDim.x >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per = H / kKBlock / W;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const char* wgt;
  const char* wup;
  if (shared) {
    wgt = static_cast<const char*>(gw.sh_gate);
    wup = static_cast<const char*>(gw.sh_up);
  } else {
    wgt = static_cast<const char*>(gw.gate_up) + static_cast<int64_t>(g) * 2 * gw.I * H * 2;
    wup = wgt + static_cast<int64_t>(gw.I) * H * 2;
  }
  const char* abase[2] = {wgt + static_cast<int64_t>(c0) * H * 2,
                          wup + static_cast<int64_t>(c0) * H * 2};
  const uint32_t aoff = static_cast<uint32_t>((q * H + 8 * r) * 2);
  for (int p0 = 16 * TT * slice; p0 < n; p0 += 16 * TT * nslices) {
    const uint16_t* bp[TT][4];
#pragma unroll
    for (int j = 0; j < TT; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + 16 * j + 4 * u + q, n - 1);   // past n: a real row, not stored
        const int tok = shared ? p : toks[p];
        bp[j][u] = x + static_cast<int64_t>(tok) * H + 8 * r;
      }
    f32x4 acc[2][TT];
    split_dot<TT, MAXB>(lds + wv * 256, abase, 4 * H * 2, aoff, bp, wv * per, per, acc);
    split_publish<TT>(lds, wv, acc);
    for (int t = threadIdx.x; t < 64 * TT; t += blockDim.x) {   // (token tile j, lane)
      const int j = t >> 6;
      const int p = p0 + 16 * j + r;
      const f32x4 gs = split_sum<TT>(lds, W, 0, j, lane);
      const f32x4 us = split_sum<TT>(lds, W, 1, j, lane);
      if (p < n) {
        float a[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) a[v] = silu(gs[v]) * us[v];
        u32x2 pk = {pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
        *reinterpret_cast<u32x2*>(act + static_cast<int64_t>(row0 + p) * act_ld + c0 + 4 * q) = pk;
      }
    }
    __syncthreads();   // partial sums read before the next pass reuses the slots
  }
}

// A launch planned for two token tiles per pass runs a group of at most 16 rows (one tile)
// with the one-tile pass instead, so the second tile's token loads and MFMAs, all padding, are
// not issued (Qwen3-30B-A3B T=192 213.5 -> 211.1 us, T=256 227.9 -> 226.1 us). Its k-blocks
// still come one per chunk: two per chunk, as the one-tile plan loads them, made the whole
// launch slower (gate_up at T=256 144 -> 153 us).
template <int TT, int MAXB>
__device__ __forceinline__ void gate_up_rows(const GroupWeights& gw, const uint16_t* __restrict__ x,
                                             int g, int n, int row0, const int32_t* toks,
                                             int slice, int nslices, int act_ld,
                                             uint16_t* __restrict__ act, u32x4* lds) {
  if constexpr (TT == 2) {
    if (n <= 16 && nslices == 1) {
      gate_up_group<1, 1>(gw, x, g, n, row0, toks, slice, nslices, act_ld, act, lds);
      return;
    }
  }
  gate_up_group<TT, MAXB>(gw, x, g, n, row0, toks, slice, nslices, act_ld, act, lds);
}

template <int TT, int MAXB>
__global__ __launch_bounds__(64 * kSplitMaxWaves) void gate_up_bf16_kernel(
    GroupWeights gw, const uint16_t* __restrict__ x, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_tok, int T,
    int shared_extra, int act_ld, uint16_t* __restrict__ act) {
  const GroupSlice gs = group_slice(gw, shared_extra, counts);
  if (gs.g < 0) return;
  const bool shared = gs.g == gw.E;
  const int n = shared ? T : counts[gs.g];
  const int row0 = shared ? gw.sh_row0 : offsets[gs.g];
  __shared__ u32x4 lds[split_lds_u4<TT>()];
  gate_up_rows<TT, MAXB>(gw, x, gs.g, n, row0, shared ? nullptr : perm_tok + row0, gs.slice,
                         gs.nslices, act_ld, act, lds);
}

// Rows of routed group g from the selected experts idx [T][k] (int32, every id in [0, E)), in
// the order the permutation builds (within an expert slot-major: (s, t) ascending;
// permute.hip): row count n, first row row0 and toks[p], the token of row p. Thread t takes
// token t (T <= threads): it loads the token's k ids and finds the slot s_t holding g, if any
// (a token selects an expert at most once). Its rank is then the tokens with g in a lower
// slot plus the lower tokens with g in slot s_t: per slot one ballot per wave, the wave
// counts through LDS. The workgroups of channel block 0 store the group's perm_tok,
// perm_slot and inv entries, workgroup (0, 0) the counts and offsets of every expert (an LDS
// histogram). Every thread of the workgroup must call it. KMAX >= k.
template <int KMAX>
__device__ __forceinline__ void group_rows(const int32_t* __restrict__ idx, int T, int k, int E,
                                           int g, const PermOut& po, int& n, int& row0,
                                           int* toks) {
  __shared__ int s_hist[1024];
  __shared__ int s_cnt[kSplitMaxWaves][KMAX + 1];     // per wave: tokens with g per slot, ids < g
  const int bd = blockDim.x, tid = threadIdx.x, lane = lane_id(), wv = tid >> 6;
  const int nw = bd >> 6;
  const bool lead = blockIdx.x == 0 && blockIdx.y == 0;
  if (lead)
    for (int e = tid; e < E; e += bd) s_hist[e] = 0;
  const int t = min(tid, T - 1);                         // threads past T re-read token T-1
  int ev[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) ev[j] = idx[t * k + min(j, k - 1)];   // unconditional loads
  if (lead) __syncthreads();                             // histogram cleared
  const bool own = tid < T;
  int slot = -1, lt = 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const bool ok = own && j < k;
    if (ok && ev[j] == g) slot = j;
    lt += ok && ev[j] < g;
    if (lead && ok) atomicAdd(&s_hist[ev[j]], 1);
  }
  uint64_t mine = 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= k) break;
    const uint64_t m = __ballot(slot == j);
    if (slot == j) mine = m;
    if (lane == 0) s_cnt[wv][j] = __popcll(m);
  }
  const int wlt = wave_sum_i32(lt);
  if (lane == 0) s_cnt[wv][KMAX] = wlt;
  __syncthreads();
  // lane j < k: slot j's tokens in all waves (col) and in the waves before this one (pre);
  // lane KMAX: the ids below g
  int col = 0, pre = 0;
  if (lane < k || lane == KMAX) {
    for (int w = 0; w < nw; ++w) {
      const int c = s_cnt[w][lane];
      col += c;
      pre += w < wv ? c : 0;
    }
  }
  row0 = __shfl(col, KMAX, kWave);
  const int cin = lane < k ? col : 0;
  int base = cin;                                        // inclusive prefix over the slots
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    const int u = __shfl_up(base, o, kWave);
    if (lane >= o) base += u;
  }
  n = __shfl(base, 15, kWave);
  base -= cin;                                           // tokens with g in lower slots
  const int sl = slot < 0 ? 0 : slot;
  const int rank = __shfl(base, sl, kWave) + __shfl(pre, sl, kWave);
  if (slot >= 0) {
    const int p = rank + mask_rank(mine);
    toks[p] = t;
    if (blockIdx.x == 0) {
      po.perm_tok[row0 + p] = t;
      po.perm_slot[row0 + p] = slot;
      po.inv[t * k + slot] = row0 + p;
    }
  }
  if (lead) {
    __syncthreads();                                     // histogram complete
    if (wv == 0) {
      // counts and offsets of every expert: lane l scans experts [l * per, (l + 1) * per)
      const int per = (E + kWave - 1) / kWave;
      const int lo = min(E, lane * per), hi = min(E, lo + per);
      int local = 0;
      for (int e = lo; e < hi; ++e) local += s_hist[e];
      int run = local;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int u = __shfl_up(run, o, kWave);
        if (lane >= o) run += u;
      }
      const int tot = run;
      run -= local;
      for (int e = lo; e < hi; ++e) {
        const int c = s_hist[e];
        po.counts[e] = c;
        po.offsets[e] = run;
        run += c;
      }
      if (lane == kWave - 1) po.offsets[E] = tot;
    }
  }
  __syncthreads();                                       // toks complete
}

template <int TT, int MAXB, int KMAX>
__global__ __launch_bounds__(64 * kSplitMaxWaves) void gate_up_bf16_perm_kernel(
    GroupWeights gw, const uint16_t* __restrict__ x, const int32_t* __restrict__ idx, PermOut po,
    int T, int k, int shared_extra, int act_ld, uint16_t* __restrict__ act) {
  __shared__ int toks[kFusedPermTokens];
  const GroupSlice gs = group_slice(gw, shared_extra, nullptr);   // hit_rows == 0
  if (gs.g < 0) return;
  int n, row0;
  if (gs.g == gw.E) {
    n = T;
    row0 = gw.sh_row0;
  } else {
    group_rows<KMAX>(idx, T, k, gw.E, gs.g, po, n, row0, toks);
  }
  __shared__ u32x4 lds[split_lds_u4<TT>()];
  gate_up_rows<TT, MAXB>(gw, x, gs.g, n, row0, toks, gs.slice, gs.nslices, act_ld, act, lds);
}

// The routing of a batch of T <= kInlineRouteTokens tokens with T*k <= kInlineRouteEntries,
// redone by every workgroup of the routed gate_up launch in place of the route and
// permutation kernels: the selection of route_topk (route_token, one wave per token), then
// this workgroup's group in the order the permutation builds (experts ascending, within an
// expert slot-major: entry v = s*T + t; permute.hip). Returns the group of workgroup row
// blockIdx.y (with hit_rows the y-th expert that received tokens; the shared expert after the
// routed rows; -1 for none) with its row count n, first row row0 and tokens toks[0 .. n).
// The workgroups of channel block 0 store their group's perm_tok, perm_slot and inv entries;
// workgroup (0, 0) also idx, topw, sgate, counts and offsets, so the later kernels and the
// workspace regions hold what the two kernels would have written.
template <int EPL>
__device__ __forceinline__ int inline_route(const GroupWeights& gw, const SmallRoute& rt,
                                            const uint16_t* __restrict__ x, int T, int& n_out,
                                            int& row0_out, int* toks) {
  __shared__ int s_idx[kInlineRouteEntries];   // token-major: [t * k + s]
  __shared__ int s_cnt[1024];                  // per expert (workgroup (0, 0) only)
  __shared__ unsigned long long s_hit[16];     // experts with tokens, E <= 1024 bits
  __shared__ int s_res[3];
  const int E = gw.E, k = rt.k, V = T * k;
  const int W = blockDim.x >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id();
  const bool lead = blockIdx.x == 0 && blockIdx.y == 0;
  if (lead)
    for (int e = threadIdx.x; e < E; e += blockDim.x) s_cnt[e] = 0;
  if (threadIdx.x < 16) s_hit[threadIdx.x] = 0ull;
  for (int t = wv; t < T; t += W)                       // the same for the whole wave
    route_token<EPL>(rt.logits, rt.bias, x, rt.w_sg, t, E, gw.H, k, s_idx, 4,
                     lead ? rt.topw : nullptr, lead ? rt.sgate : nullptr);
  __syncthreads();
  // wave 0, lane v: entry v = s*T + t
  const bool valid = wv == 0 && lane < V;
  const int s = lane / T, t = lane - (lane / T) * T;
  const int e = valid ? s_idx[t * k + s] : 0;
  if (valid) {
    atomicOr(&s_hit[e >> 6], 1ull << (e & 63));
    if (lead) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();
  if (wv == 0) {
    const int rows = routed_rows(gw), y = blockIdx.y;
    int g = -1;
    if (y >= rows) {
      g = E;
    } else if (gw.hit_rows == 0) {
      g = gw.g0 + y;
    } else {
      // the y-th set bit of the hit mask: word by a prefix sum over 16 lanes, then the bit
      const unsigned long long word = lane < 16 ? s_hit[lane] : 0ull;
      const int c = __popcll(word);
      int incl = c;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int u = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += u;
      }
      const uint64_t who = __ballot(lane < 16 && y >= incl - c && y < incl);
      if (who != 0) {
        const int wl = __builtin_ctzll(who);
        const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(word), wl);
        const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(word >> 32), wl);
        const unsigned long long wd = (static_cast<unsigned long long>(hi) << 32) | lo;
        const int rank = y - (__builtin_amdgcn_readlane(incl, wl) - __popcll(wd));
        const unsigned long long below = wd & ((1ull << lane) - 1ull);
        const uint64_t sel = __ballot(((wd >> lane) & 1ull) != 0 && __popcll(below) == rank);
        g = wl * 64 + __builtin_ctzll(sel);
      }
    }
    int n = 0, row0 = 0;
    if (g >= 0 && g < E) {
      const uint64_t eq = __ballot(valid && e == g);
      n = __popcll(eq);
      row0 = __popcll(__ballot(valid && e < g));
      if (valid && e == g) {
        const int p = __popcll(eq & ((1ull << lane) - 1ull));
        toks[p] = t;
        if (blockIdx.x == 0) {
          rt.perm_tok[row0 + p] = t;
          rt.perm_slot[row0 + p] = s;
          rt.inv[t * k + s] = row0 + p;
        }
      }
    }
    if (lead) {
      if (valid) rt.idx[t * k + s] = e;
      // counts and offsets of every expert: lane l scans experts [l * per, (l + 1) * per)
      const int per = (E + kWave - 1) / kWave;
      const int lo = min(E, lane * per), hi = min(E, lo + per);
      int local = 0;
      for (int e2 = lo; e2 < hi; ++e2) local += s_cnt[e2];
      int incl = local;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int u = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += u;
      }
      int run = incl - local;
      for (int e2 = lo; e2 < hi; ++e2) {
        const int c2 = s_cnt[e2];
        rt.counts[e2] = c2;
        rt.offsets[e2] = run;
        run += c2;
      }
      if (lane == kWave - 1) rt.offsets[E] = incl;
    }
    if (lane == 0) {
      s_res[0] = g;
      s_res[1] = n;
      s_res[2] = row0;
    }
  }
  __syncthreads();
  n_out = s_res[1];
  row0_out = s_res[2];
  return s_res[0];
}

template <int MAXB, int EPL>
__global__ __launch_bounds__(64 * kSplitMaxWaves) void gate_up_bf16_routed_kernel(
    GroupWeights gw, const uint16_t* __restrict__ x, SmallRoute rt, int T, int shared_extra,
    int act_ld, uint16_t* __restrict__ act) {
  __shared__ int toks[kInlineRouteTokens];
  int n, row0;
  const int g = inline_route<EPL>(gw, rt, x, T, n, row0, toks);
  if (g < 0) return;
  int slice = 0, nslices = 1;
  if (g == gw.E) {
    slice = blockIdx.y - routed_rows(gw);
    nslices = shared_extra + 1;
    n = T;
    row0 = gw.sh_row0;
  }
  __shared__ u32x4 lds[split_lds_u4<1>()];
  gate_up_group<1, MAXB>(gw, x, g, n, row0, toks, slice, nslices, act_ld, act, lds);
}

hipError_t launch_gate_up_bf16(const GroupWeights& gw, const void* x, const int32_t* counts,
                               const int32_t* offsets, const int32_t* perm_tok, int64_t T,
                               int k, int act_ld, void* act, hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  auto go = [&]<int TT>() {
    const int extra = shared_extra_rows(gw, T, 16 * TT);
    const dim3 grid(Imax / 16, grid_groups(gw) + extra);
    const SplitPlan plan = split_plan(gw.H / kKBlock, TT, false);
    return with_maxb<TT>(plan, [&]<int TT_, int MAXB>() {
      gate_up_bf16_kernel<TT_, MAXB><<<grid, 64 * plan.waves, 0, s>>>(
          gw, static_cast<const uint16_t*>(x), counts, offsets, perm_tok, static_cast<int>(T),
          extra, act_ld, static_cast<uint16_t*>(act));
      return hipGetLastError();
    });
  };
  switch (pick_tt(gw, T, k)) {
    case 1: return go.template operator()<1>();
    case 2: return go.template operator()<2>();
    default: return go.template operator()<4>();
  }
}

bool inline_route_supported(int64_t T, int k, int E) {
  return T >= 1 && T <= kInlineRouteTokens && T * k <= kInlineRouteEntries && E <= 1024;
}

hipError_t launch_gate_up_bf16_routed(const GroupWeights& gw, const void* x, const SmallRoute& rt,
                                      int64_t T, int act_ld, void* act, hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  const int extra = shared_extra_rows(gw, T, 16);
  const dim3 grid(Imax / 16, grid_groups(gw) + extra);
  const SplitPlan plan = split_plan(gw.H / kKBlock, 1, false);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* a = static_cast<uint16_t*>(act);
  const int Ti = static_cast<int>(T);
  return with_maxb<1>(plan, [&]<int TT_, int MAXB>() {
#define LBMOE_ROUTED(EPL) \
  gate_up_bf16_routed_kernel<MAXB, EPL><<<grid, 64 * plan.waves, 0, s>>>(gw, xx, rt, Ti, extra, act_ld, a)
    if (gw.E <= 64) LBMOE_ROUTED(1);
    else if (gw.E <= 128) LBMOE_ROUTED(2);
    else if (gw.E <= 256) LBMOE_ROUTED(4);
    else if (gw.E <= 512) LBMOE_ROUTED(8);
    else LBMOE_ROUTED(16);
#undef LBMOE_ROUTED
    return hipGetLastError();
  });
}

bool gate_up_perm_supported(const GroupWeights& gw, int64_t T, int k) {
  if (T < 1 || T > kFusedPermTokens || T * k < gw.E || gw.E > 1024 || gw.hit_rows != 0 || k > 16)
    return false;
  const SplitPlan plan = split_plan(gw.H / kKBlock, pick_tt(gw, T, k), false);
  return T <= 64 * plan.waves;                           // one token per thread
}

hipError_t launch_gate_up_bf16_perm(const GroupWeights& gw, const void* x, const int32_t* idx,
                                    const PermOut& po, int64_t T, int k, int act_ld, void* act,
                                    hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  auto go = [&]<int TT>() {
    const int extra = shared_extra_rows(gw, T, 16 * TT);
    const dim3 grid(Imax / 16, grid_groups(gw) + extra);
    const SplitPlan plan = split_plan(gw.H / kKBlock, TT, false);
    return with_maxb<TT>(plan, [&]<int TT_, int MAXB>() {
      const auto* xx = static_cast<const uint16_t*>(x);
      auto* a = static_cast<uint16_t*>(act);
      const int Ti = static_cast<int>(T);
      if (k <= 8)
        gate_up_bf16_perm_kernel<TT_, MAXB, 8><<<grid, 64 * plan.waves, 0, s>>>(
            gw, xx, idx, po, Ti, k, extra, act_ld, a);
      else
        gate_up_bf16_perm_kernel<TT_, MAXB, 16><<<grid, 64 * plan.waves, 0, s>>>(
            gw, xx, idx, po, Ti, k, extra, act_ld, a);
      return hipGetLastError();
    });
  };
  switch (pick_tt(gw, T, k)) {
    case 1: return go.template operator()<1>();
    case 2: return go.template operator()<2>();
    default: return go.template operator()<4>();
  }
}

// ---- down projection ---------------------------------------------------------------------
// Workgroup (row block hb, group g): output columns [32hb, 32hb+32) of H for every token row of
// the group: out[row, h] = bf16(act[row, :Ig] . Wd_g[h, :Ig]) (qwen3_5.py:837, :868, :917).
// Output columns [h0, h0 + 32) of group g's n rows from row0 on (K = Ig), TT token tiles per
// pass; the passes slice, slice + nslices, ... of the group.
template <int TT, int MAXB>
__device__ __forceinline__ void down_group(const GroupWeights& gw, const uint16_t* __restrict__ act,
                                           int act_ld, int g, int Ig, int n, int row0, int slice,
                                           int nslices, uint16_t* __restrict__ out, u32x4* lds) {
  const bool shared = g == gw.E;
  const int H = gw.H;
  const int h0 = blockIdx.x * 32;
  const int W = blockDim.x >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per = Ig / kKBlock / W;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const char* wd = shared ? static_cast<const char*>(gw.sh_down)
                          : static_cast<const char*>(gw.down) + static_cast<int64_t>(g) * H * gw.I * 2;
  const char* abase[2] = {wd + static_cast<int64_t>(h0) * Ig * 2,
                          wd + static_cast<int64_t>(h0 + 16) * Ig * 2};
  const uint32_t aoff = static_cast<uint32_t>((q * Ig + 8 * r) * 2);
  for (int p0 = 16 * TT * slice; p0 < n; p0 += 16 * TT * nslices) {
    const uint16_t* bp[TT][4];
#pragma unroll
    for (int j = 0; j < TT; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + 16 * j + 4 * u + q, n - 1);   // past n: a real row, not stored
        bp[j][u] = act + static_cast<int64_t>(row0 + p) * act_ld + 8 * r;
      }
    f32x4 acc[2][TT];
    split_dot<TT, MAXB>(lds + wv * 256, abase, 4 * Ig * 2, aoff, bp, wv * per, per, acc);
    split_publish<TT>(lds, wv, acc);
    for (int t = threadIdx.x; t < 2 * 64 * TT; t += blockDim.x) {   // (tile i, token tile j, lane)
      const int i = t >> 6 & 1, j = t >> 7;
      const int p = p0 + 16 * j + r;
      const f32x4 v = split_sum<TT>(lds, W, i, j, lane);
      if (p < n) {
        u32x2 pk = {pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
        *reinterpret_cast<u32x2*>(out + static_cast<int64_t>(row0 + p) * H + h0 + 16 * i + 4 * q) = pk;
      }
    }
    __syncthreads();   // partial sums read before the next pass reuses the slots
  }
}

// Workgroup (row block hb, group g): output columns [32hb, 32hb+32) of H for every token row of
// the group: out[row, h] = bf16(act[row, :Ig] . Wd_g[h, :Ig]) (qwen3_5.py:837, :868, :917). A
// launch planned for two token tiles runs groups of at most 16 rows with the one-tile pass
// (T=192 down 72.1 -> 70.3 us).
template <int TT, int MAXB>
__global__ __launch_bounds__(64 * kSplitMaxWaves) void down_bf16_kernel(
    GroupWeights gw, const uint16_t* __restrict__ act, int act_ld,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets, int T,
    int shared_extra, int width, uint16_t* __restrict__ out) {
  const GroupSlice gs = group_slice(gw, shared_extra, counts);
  const int g = gs.g;
  if (g < 0) return;
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  if (Ig != width) return;          // groups of another width run in their own launch
  const int n = shared ? T : counts[g];
  if (n == 0) return;
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  __shared__ u32x4 lds[split_lds_u4<TT>()];
  if constexpr (TT == 2) {
    if (n <= 16 && gs.nslices == 1) {
      down_group<1, 1>(gw, act, act_ld, g, Ig, n, row0, gs.slice, gs.nslices, out, lds);
      return;
    }
  }
  down_group<TT, MAXB>(gw, act, act_ld, g, Ig, n, row0, gs.slice, gs.nslices, out, lds);
}

hipError_t launch_down_bf16(const GroupWeights& gw, const void* act, int act_ld,
                            const int32_t* counts, const int32_t* offsets, int64_t T, int k,
                            void* out, hipStream_t s) {
  const int tt = pick_tt(gw, T, k);
  auto go = [&](int K) {
    auto launch = [&]<int TT>() {
      const int extra = shared_extra_rows(gw, T, 16 * TT);
      const dim3 grid(gw.H / 32, grid_groups(gw) + extra);
      const SplitPlan plan = split_plan(K / kKBlock, TT, true);
      return with_maxb<TT>(plan, [&]<int TT_, int MAXB>() {
        down_bf16_kernel<TT_, MAXB><<<grid, 64 * plan.waves, 0, s>>>(
            gw, static_cast<const uint16_t*>(act), act_ld, counts, offsets, static_cast<int>(T),
            extra, K, static_cast<uint16_t*>(out));
        return hipGetLastError();
      });
    };
    switch (tt) {
      case 1: return launch.template operator()<1>();
      case 2: return launch.template operator()<2>();
      default: return launch.template operator()<4>();
    }
  };
  // Routed experts (width I) and the shared expert (width Is) each get a launch planned for
  // their width; a group whose width differs from the launch's exits at once.
  const bool has_routed = gw.g0 < gw.E;
  const bool has_shared = gw.g0 + gw.groups > gw.E;
  hipError_t e = hipSuccess;
  if (has_routed) e = go(gw.I);
  if (e == hipSuccess && has_shared && (!has_routed || gw.Is != gw.I)) e = go(gw.Is);
  return e;
}

}  // namespace lbmoe
