// fp8 (OCP e4m3fn) quantisation kernels. The reference has no fp8 path; these define the
// quantised variant: weights per 128x128 block and activations per (row, 128 channels), with
// scale = amax / 448 (an all-zero block gets scale 1) and code = e4m3(value / scale) rounded
// to nearest even and saturated to +-448.
#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

// One 256-thread workgroup per 128x128 block; thread i covers row i/2, 64 columns.
__global__ __launch_bounds__(256) void quant_blocks_kernel(const uint16_t* __restrict__ w,
                                                           int N, int K,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale) {
  __shared__ float red[4];
  const int nbk = K / 128, nbn = N / 128;
  const int64_t blk = blockIdx.x;
  const int64_t b = blk / (static_cast<int64_t>(nbn) * nbk);
  const int rem = static_cast<int>(blk - b * nbn * nbk);
  const int bn = rem / nbk, bk = rem - bn * nbk;
  const int row = bn * 128 + (threadIdx.x >> 1);
  const int col = bk * 128 + (threadIdx.x & 1) * 64;
  const int64_t base = (b * N + row) * static_cast<int64_t>(K) + col;
  u32x4 v[8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = ld16(w + base + 8 * i);
#pragma unroll
    for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fmaxf(fabsf(bf_lo(v[i][j])), fabsf(bf_hi(v[i][j]))));
  }
  amax = wave_max(amax);
  if (lane_id() == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fp8_scale_of(amax);
  if (threadIdx.x == 0) scale[blk] = s;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t lo = v[i + h][2 * j], hi = v[i + h][2 * j + 1];
        o[2 * h + j] = e4m3x4(bf_lo(lo) / s, bf_hi(lo) / s, bf_lo(hi) / s, bf_hi(hi) / s);
      }
    }
    *reinterpret_cast<u32x4*>(q + base + 8 * i) = o;
  }
}

hipError_t launch_quant_blocks_fp8(const void* w, int64_t batch, int N, int K, void* q,
                                   float* scale, hipStream_t s) {
  const int64_t nblocks = batch * (N / 128) * (K / 128);
  quant_blocks_kernel<<<static_cast<unsigned>(nblocks), 256, 0, s>>>(
      static_cast<const uint16_t*>(w), N, K, static_cast<uint8_t*>(q), scale);
  return hipGetLastError();
}

// 16 lanes per (row, 128-channel group), 8 channels per lane (16-byte loads, 8-byte stores);
// the group's amax is reduced over its 16 lanes.
constexpr int kGroupsPerBlock = 16;
__global__ __launch_bounds__(256) void quant_groups_kernel(const uint16_t* __restrict__ a,
                                                           int64_t rows, int cols, int ld,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale) {
  const int ng = cols / 128;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kGroupsPerBlock + (threadIdx.x >> 4);
  if (gid >= rows * ng) return;
  const int64_t row = gid / ng;
  const int grp = static_cast<int>(gid - row * ng);
  const int sub = threadIdx.x & 15;
  float sc;
  const u32x2 c = quant_group16(ld16(a + row * ld + grp * 128 + 8 * sub), sc);
  if (sub == 0) scale[row * ng + grp] = sc;
  *reinterpret_cast<u32x2*>(q + row * cols + grp * 128 + 8 * sub) = c;
}

hipError_t launch_quant_groups_fp8(const void* a, int64_t rows, int cols, int ld, void* q,
                                   float* scale, hipStream_t s) {
  const int64_t groups = rows * (cols / 128);
  if (groups == 0) return hipSuccess;
  quant_groups_kernel<<<static_cast<unsigned>((groups + kGroupsPerBlock - 1) / kGroupsPerBlock),
                        256, 0, s>>>(
      static_cast<const uint16_t*>(a), rows, cols, ld, static_cast<uint8_t*>(q), scale);
  return hipGetLastError();
}

}  // namespace lbmoe

// ---- fp8 weight-streaming GEMMs -----------------------------------------------------------
// One wave owns 16 weight rows per tile (RA tiles) and streams them once per pass over its
// group's tokens, loading 4 rows x 256 contiguous bytes per instruction and transposing through
// a per-wave LDS scratch, as the bf16 decode GEMMs do (stream_gemm.hip) but without their
// split-K workgroups: an fp8 row block carries half the bytes, and split across waves the
// per-workgroup overhead outweighed the burst (measured slower). With one
// byte per element a 256-byte row segment is 256 k; it holds two 128-k scale blocks, each
// one v_mfma_scale_f32_16x16x128_f8f6f4 (OCP e4m3 operands, unit E8M0 block scales): lane
// (r, q) supplies 32 bytes k = 128c + 32q .. +32 of row r. The block product is scaled by
// w_scale(row block, k block) * a_scale(token, k block) and added to the fp32 accumulator.
namespace lbmoe {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
constexpr int kF8Block = 256;   // k (= bytes) per streamed block

// Loads the 256-byte k-block at byte k0 of the RA weight tiles and the TT token tiles. abase[i]
// is tile i's wave-uniform first row, astep the uniform byte step of 4 rows and aoff this lane's
// 32-bit offset (row q of each 4-row group, 16-byte chunk r), so the weight loads take the
// scalar-base form; the token rows are gathered per lane.
template <int RA, int TT>
__device__ __forceinline__ void f8_load(const uint8_t* const (&abase)[RA], int astep, uint32_t aoff,
                                        const uint8_t* const (&bp)[TT][4], int k0,
                                        u32x4 (&a)[RA][4], u32x4 (&b)[TT][4]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) a[i][u] = ld16_stream(abase[i] + (k0 + u * astep) + aoff);
#pragma unroll
  for (int j = 0; j < TT; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) b[j][u] = ld16(bp[j][u] + k0);
}

__device__ __forceinline__ i32x8_t cat8(u32x4 lo, u32x4 hi) {
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// ws[i][c]: weight scale of tile i for scale block c of this k-block (wave-uniform);
// xsc[j][c]: scale of this lane's token column in tile j.
template <int RA, int TT>
__device__ __forceinline__ void f8_mma(u32x4* __restrict__ lds, const u32x4 (&a)[RA][4],
                                       const u32x4 (&b)[TT][4], const float (&ws)[RA][2],
                                       const float (&xsc)[TT][2], f32x4 (&acc)[RA][TT]) {
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
  for (int c = 0; c < 2; ++c) {
    const int j0 = 8 * c + 2 * q;
    i32x8_t fa[RA], fb[TT];
#pragma unroll
    for (int i = 0; i < RA; ++i)
      fa[i] = cat8(lds[(16 * i + r) * 16 + (j0 ^ r)], lds[(16 * i + r) * 16 + ((j0 + 1) ^ r)]);
#pragma unroll
    for (int j = 0; j < TT; ++j)
      fb[j] = cat8(lds[(16 * (RA + j) + r) * 16 + (j0 ^ r)],
                   lds[(16 * (RA + j) + r) * 16 + ((j0 + 1) ^ r)]);
#pragma unroll
    for (int i = 0; i < RA; ++i)
#pragma unroll
      for (int j = 0; j < TT; ++j) {
        const f32x4 p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            fa[i], fb[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        acc[i][j] += p * (ws[i][c] * xsc[j][c]);
      }
  }
}

// acc += the products over K (a multiple of 256). PREFETCH: the next k-block's loads go out
// before this one's MFMAs, into a second set of registers (gate_up, 8 k-blocks at H = 2048);
// else one k-block at a time (down, 2 k-blocks at I = 512), which takes the kernel from 192
// to 136 VGPRs, so each SIMD holds three waves' loads instead of two's: E=512 fp8 T=128 down
// 91.0 -> 85.9 us; for gate_up the prefetch is worth more (151.5 against 153.3 us).
// The k-blocks add up in the same order either way. wsp[i]: tile i's row of block scales
// (K/128 entries); xsp[j]: the lane's token scales.
template <int RA, int TT, bool PREFETCH>
__device__ __forceinline__ void f8_dot(u32x4* __restrict__ lds, const uint8_t* const (&abase)[RA],
                                       int astep, uint32_t aoff, const uint8_t* const (&bp)[TT][4],
                                       const float* const (&wsp)[RA], const float* const (&xsp)[TT],
                                       int K, f32x4 (&acc)[RA][TT]) {
  u32x4 a[RA][4], b[TT][4];
  if constexpr (PREFETCH) f8_load<RA, TT>(abase, astep, aoff, bp, 0, a, b);
  for (int kb = 0; kb < K; kb += kF8Block) {
    u32x4 an[RA][4], bn[TT][4];
    if constexpr (PREFETCH) {
      if (kb + kF8Block < K) f8_load<RA, TT>(abase, astep, aoff, bp, kb + kF8Block, an, bn);
    } else {
      f8_load<RA, TT>(abase, astep, aoff, bp, kb, a, b);
    }
    const int sb = kb / 128;
    float ws[RA][2], xsc[TT][2];
#pragma unroll
    for (int i = 0; i < RA; ++i) {
      ws[i][0] = wsp[i][sb];
      ws[i][1] = wsp[i][sb + 1];
    }
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      xsc[j][0] = xsp[j][sb];
      xsc[j][1] = xsp[j][sb + 1];
    }
    f8_mma<RA, TT>(lds, a, b, ws, xsc, acc);
    if constexpr (PREFETCH) {
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

template <int RA, int TT>
__device__ __forceinline__ void zero_acc8(f32x4 (&acc)[RA][TT]) {
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// gate_up: wave (channel block cb, group g) -> act[row, 16cb .. 16cb+15] (bf16).
template <int TT>
__global__ __launch_bounds__(64) void gate_up_fp8_kernel(GroupWeights gw, const uint8_t* __restrict__ xq,
                                                         const float* __restrict__ xs,
                                                         const int32_t* __restrict__ counts,
                                                         const int32_t* __restrict__ offsets,
                                                         const int32_t* __restrict__ perm_tok,
                                                         int T, int shared_extra, int act_ld,
                                                         uint16_t* __restrict__ act) {
  __shared__ u32x4 lds[(2 + TT) * 256];
  const GroupSlice gs = group_slice(gw, shared_extra, counts);
  const int g = gs.g;
  if (g < 0) return;
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int c0 = blockIdx.x * 16;
  if (c0 >= Ig) return;
  const int n = shared ? T : counts[g];
  if (n == 0) return;
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  const int H = gw.H, nkb = H / 128;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const uint8_t* wgt;
  const uint8_t* wup;
  const float* sg;
  const float* su;
  if (shared) {
    wgt = static_cast<const uint8_t*>(gw.sh_gate);
    wup = static_cast<const uint8_t*>(gw.sh_up);
    sg = gw.sh_gate_scale + static_cast<int64_t>(c0 / 128) * nkb;
    su = gw.sh_up_scale + static_cast<int64_t>(c0 / 128) * nkb;
  } else {
    wgt = static_cast<const uint8_t*>(gw.gate_up) + static_cast<int64_t>(g) * 2 * gw.I * H;
    wup = wgt + static_cast<int64_t>(gw.I) * H;
    const float* s0 = gw.gate_up_scale + static_cast<int64_t>(g) * (2 * gw.I / 128) * nkb;
    sg = s0 + static_cast<int64_t>(c0 / 128) * nkb;
    su = s0 + static_cast<int64_t>((gw.I + c0) / 128) * nkb;
  }
  const uint8_t* abase[2] = {wgt + static_cast<int64_t>(c0) * H, wup + static_cast<int64_t>(c0) * H};
  const uint32_t aoff = static_cast<uint32_t>(q * H + 16 * r);
  const float* wsp[2] = {sg, su};
  for (int p0 = 16 * TT * gs.slice; p0 < n; p0 += 16 * TT * gs.nslices) {
    const uint8_t* bp[TT][4];
    const float* xsp[TT];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + 16 * j + 4 * u + q, n - 1);   // past n: a real row, not stored
        const int tok = shared ? p : perm_tok[row0 + p];
        bp[j][u] = xq + static_cast<int64_t>(tok) * H + 16 * r;
      }
      const int pc = min(p0 + 16 * j + r, n - 1);          // this lane's accumulator column
      const int tc = shared ? pc : perm_tok[row0 + pc];
      xsp[j] = xs + static_cast<int64_t>(tc) * nkb;
    }
    f32x4 acc[2][TT];
    zero_acc8(acc);
    f8_dot<2, TT, true>(lds, abase, 4 * H, aoff, bp, wsp, xsp, H, acc);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int p = p0 + 16 * j + r;
      if (p >= n) continue;
      float a[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) a[v] = silu(acc[0][j][v]) * acc[1][j][v];
      *reinterpret_cast<u32x2*>(act + static_cast<int64_t>(row0 + p) * act_ld + c0 + 4 * q) =
          u32x2{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
    }
  }
}

// down: wave (row block hb of 32, group g) -> out[row, 32hb .. 32hb+31] (bf16).
template <int TT>
__global__ __launch_bounds__(64) void down_fp8_kernel(GroupWeights gw, const uint8_t* __restrict__ aq,
                                                      const float* __restrict__ as, int act_ld,
                                                      const int32_t* __restrict__ counts,
                                                      const int32_t* __restrict__ offsets, int T,
                                                      int shared_extra, uint16_t* __restrict__ out) {
  __shared__ u32x4 lds[(2 + TT) * 256];
  const GroupSlice gs = group_slice(gw, shared_extra, counts);
  const int g = gs.g;
  if (g < 0) return;
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int n = shared ? T : counts[g];
  if (n == 0) return;
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  const int H = gw.H, h0 = blockIdx.x * 32;
  const int nkb = Ig / 128, nsa = act_ld / 128;
  const int lane = lane_id(), r = lane & 15, q = lane >> 4;
  const uint8_t* wd;
  const float* sd;
  if (shared) {
    wd = static_cast<const uint8_t*>(gw.sh_down);
    sd = gw.sh_down_scale + static_cast<int64_t>(h0 / 128) * nkb;
  } else {
    wd = static_cast<const uint8_t*>(gw.down) + static_cast<int64_t>(g) * H * gw.I;
    sd = gw.down_scale + (static_cast<int64_t>(g) * (H / 128) + h0 / 128) * nkb;
  }
  const uint8_t* abase[2] = {wd + static_cast<int64_t>(h0) * Ig,
                             wd + static_cast<int64_t>(h0 + 16) * Ig};
  const uint32_t aoff = static_cast<uint32_t>(q * Ig + 16 * r);
  const float* wsp[2] = {sd, sd};
  for (int p0 = 16 * TT * gs.slice; p0 < n; p0 += 16 * TT * gs.nslices) {
    const uint8_t* bp[TT][4];
    const float* xsp[TT];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + 16 * j + 4 * u + q, n - 1);   // past n: a real row, not stored
        bp[j][u] = aq + static_cast<int64_t>(row0 + p) * act_ld + 16 * r;
      }
      const int pc = min(p0 + 16 * j + r, n - 1);
      xsp[j] = as + static_cast<int64_t>(row0 + pc) * nsa;
    }
    f32x4 acc[2][TT];
    zero_acc8(acc);
    f8_dot<2, TT, false>(lds, abase, 4 * Ig, aoff, bp, wsp, xsp, Ig, acc);
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int p = p0 + 16 * j + r;
      if (p >= n) continue;
      uint16_t* orow = out + static_cast<int64_t>(row0 + p) * H + h0 + 4 * q;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        *reinterpret_cast<u32x2*>(orow + 16 * i) =
            u32x2{pack_bf2(acc[i][j][0], acc[i][j][1]), pack_bf2(acc[i][j][2], acc[i][j][3])};
    }
  }
}

static int pick_tt8(const GroupWeights& gw, int64_t T, int k) {
  const double avg = gw.g0 < gw.E ? static_cast<double>(T) * k / gw.E : static_cast<double>(T);
  return avg <= 12.0 ? 1 : (avg <= 28.0 ? 2 : 4);
}

// Calls f.template operator()<TT>() for the token-tile count tt.
template <typename F>
static hipError_t with_tt8(int tt, F&& f) {
  switch (tt) {
    case 1: return f.template operator()<1>();
    case 2: return f.template operator()<2>();
    default: return f.template operator()<4>();
  }
}

hipError_t launch_gate_up_fp8(const GroupWeights& gw, const void* xq, const float* xs,
                              const int32_t* counts, const int32_t* offsets,
                              const int32_t* perm_tok, int64_t T, int k, int act_ld, void* act,
                              hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  return with_tt8(pick_tt8(gw, T, k), [&]<int TT>() {
    const int extra = shared_extra_rows(gw, T, 16 * TT);
    gate_up_fp8_kernel<TT><<<dim3(Imax / 16, grid_groups(gw) + extra), 64, 0, s>>>(
        gw, static_cast<const uint8_t*>(xq), xs, counts, offsets, perm_tok, static_cast<int>(T),
        extra, act_ld, static_cast<uint16_t*>(act));
    return hipGetLastError();
  });
}

hipError_t launch_down_fp8(const GroupWeights& gw, const void* actq, const float* acts,
                           int act_ld, const int32_t* counts, const int32_t* offsets,
                           int64_t T, int k, void* out, hipStream_t s) {
  return with_tt8(pick_tt8(gw, T, k), [&]<int TT>() {
    const int extra = shared_extra_rows(gw, T, 16 * TT);
    down_fp8_kernel<TT><<<dim3(gw.H / 32, grid_groups(gw) + extra), 64, 0, s>>>(
        gw, static_cast<const uint8_t*>(actq), acts, act_ld, counts, offsets,
        static_cast<int>(T), extra, static_cast<uint16_t*>(out));
    return hipGetLastError();
  });
}

}  // namespace lbmoe
