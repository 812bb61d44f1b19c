// LDS-tiled grouped GEMMs with fp8 (OCP e4m3) weights and activations, for prefill-sized
// batches. They take a tile list of kFp8TileTokens-token tiles from build_tiles
// (tiled_gemm.hip), deal its (token tile, weight tile) items to the XCDs in contiguous chunks
// (xcd_item), and stage operands through a global->LDS ring; the products are those of the
// fp8 streaming kernels (fp8.hip).
//
// A k-stage is 128 k = 128 bytes per row = exactly one 128-k scale block, and one
// v_mfma_scale_f32_16x16x128_f8f6f4 covers a 16 x 16 tile over the whole block (lane
// (r, q) supplies bytes 32q .. 32q+31 of row r, OCP e4m3 operands, unit E8M0 scales). The
// block product is scaled by w_scale(row block, k block) * a_scale(token, k block) and added
// to the fp32 accumulator, so no partial sums need extra registers.
// Workgroup: 4 waves in 2 x 2, tile kWM = 256 weight rows x kWT = 128 tokens; a wave owns
// 128 rows (8 tiles of 16) x 64 tokens (4 tiles of 16). Accumulator lane (r, q) of a tile
// holds token column r and rows 4q .. 4q+3, so four consecutive channels are stored together.
#include "common.hpp"
#include "internal.hpp"
#include "tiled_common.hpp"

namespace lbmoe {
namespace f8t {

typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kWM = 256;                 // weight rows per workgroup
constexpr int kWT = kFp8TileTokens;     // tokens per workgroup (the fp8 tile list's width)
constexpr int kBK = 128;                 // k (= bytes) per LDS stage
constexpr int kStages = 3;
constexpr int kWaves = 4;
constexpr int kChunks = kBK / 16;        // 16-byte chunks per LDS row
constexpr int kRowsPerLoad = 64 / kChunks;
constexpr int kALoads = kWM / kRowsPerLoad / kWaves;
constexpr int kBLoads = kWT / kRowsPerLoad / kWaves;
constexpr int kMT = kWM / 2 / 16;        // 16-row tiles per wave (weights)
constexpr int kNT = kWT / 2 / 16;        // 16-column tiles per wave (tokens)
constexpr int kStageU4 = (kWM + kWT) * kChunks;

__device__ __forceinline__ int swz(int r, int j) { return r * kChunks + (j ^ ((r >> 1) & 7)); }

__device__ __forceinline__ i32x8_t cat8(u32x4 lo, u32x4 hi) {
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                 (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

template <bool GATEUP>
__global__ __launch_bounds__(256) void tiled_fp8_kernel(
    GroupWeights gw, const uint8_t* __restrict__ src, const float* __restrict__ src_scale,
    int src_ld, const int32_t* __restrict__ offsets, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ perm_tok, const int32_t* __restrict__ tiles, int max_tiles,
    int n_wtiles, int T, uint16_t* __restrict__ dst, int dst_ld) {
  __shared__ u32x4 lds[kStages][kStageU4];
  const int logical = xcd_item(blockIdx.x, tiles[2 * max_tiles] * n_wtiles);
  if (logical < 0) return;
  const int ti = logical / n_wtiles, wt = logical - ti * n_wtiles;
  const int g = tiles[2 * ti], r0 = tiles[2 * ti + 1];
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int H = gw.H;
  const int n = shared ? T : counts[g];
  const int row0 = shared ? gw.sh_row0 : offsets[g];
  const int K = GATEUP ? H : Ig;
  const int nkb = K / 128;
  const int c0 = wt * (GATEUP ? kWM / 2 : kWM);
  if (c0 >= (GATEUP ? Ig : H)) return;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w & 1, wn = w >> 1;

  // weight rows, their block scales (rows of K/128 floats) and this thread's copy pointers
  const uint8_t* wbase;
  const uint8_t* wup = nullptr;
  const float* sw0;                      // scales of the wave's first (gate / down) block
  const float* sw1;                      // scales of the wave's up block (gate_up only)
  if (GATEUP) {
    if (shared) {
      wbase = static_cast<const uint8_t*>(gw.sh_gate);
      wup = static_cast<const uint8_t*>(gw.sh_up);
      sw0 = gw.sh_gate_scale + static_cast<int64_t>(c0 / 128) * nkb;
      sw1 = gw.sh_up_scale + static_cast<int64_t>(c0 / 128) * nkb;
    } else {
      wbase = static_cast<const uint8_t*>(gw.gate_up) + static_cast<int64_t>(g) * 2 * gw.I * H;
      wup = wbase + static_cast<int64_t>(gw.I) * H;
      const float* s0 = gw.gate_up_scale + static_cast<int64_t>(g) * (2 * gw.I / 128) * nkb;
      sw0 = s0 + static_cast<int64_t>(c0 / 128) * nkb;
      sw1 = s0 + static_cast<int64_t>((gw.I + c0) / 128) * nkb;
    }
  } else {
    const int hb = (c0 + wm * (kWM / 2)) / 128;
    if (shared) {
      wbase = static_cast<const uint8_t*>(gw.sh_down);
      sw0 = gw.sh_down_scale + static_cast<int64_t>(hb) * nkb;
    } else {
      wbase = static_cast<const uint8_t*>(gw.down) + static_cast<int64_t>(g) * H * gw.I;
      sw0 = gw.down_scale + (static_cast<int64_t>(g) * (H / 128) + hb) * nkb;
    }
    sw1 = sw0;
  }
  const int lrow = lane / kChunks, lpos = lane % kChunks;
  const uint8_t* ap[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int row = (w * kALoads + i) * kRowsPerLoad + lrow;
    const int j = lpos ^ ((row >> 1) & 7);
    const uint8_t* base = wbase;
    int grow;
    if (GATEUP) {
      const int half = row / (kWM / 2), sub = row % (kWM / 2);
      base = sub < kWM / 4 ? wbase : wup;
      grow = c0 + half * (kWM / 4) + (sub % (kWM / 4));
    } else {
      grow = c0 + row;
    }
    ap[i] = base + static_cast<int64_t>(grow) * K + 16 * j;
  }
  const uint8_t* bp[kBLoads];
#pragma unroll
  for (int i = 0; i < kBLoads; ++i) {
    const int lt = (w * kBLoads + i) * kRowsPerLoad + lrow;
    const int row = kWM + lt;
    const int j = lpos ^ ((row >> 1) & 7);
    const int p = min(r0 + lt, n - 1);   // rows past the group repeat a valid row; not stored
    const int srow = GATEUP ? (shared ? p : perm_tok[row0 + p]) : row0 + p;
    bp[i] = src + static_cast<int64_t>(srow) * src_ld + 16 * j;
  }
  // activation scale rows of this lane's accumulator columns
  const int r = lane & 15, q = lane >> 4;
  const int sa_ld = src_ld / 128;
  const float* sap[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int p = min(r0 + wn * (kWT / 2) + 16 * t + r, n - 1);
    const int srow = GATEUP ? (shared ? p : perm_tok[row0 + p]) : row0 + p;
    sap[t] = src_scale + static_cast<int64_t>(srow) * sa_ld;
  }

  f32x4 acc[kMT][kNT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int t = 0; t < kNT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  typedef __attribute__((address_space(3))) void* lds_ptr;
  auto issue = [&](int stage, int k0) {
    u32x4* buf = lds[stage];
#pragma unroll
    for (int i = 0; i < kALoads; ++i)
      __builtin_amdgcn_global_load_lds(ap[i] + k0,
                                       (lds_ptr)(buf + (w * kALoads + i) * kRowsPerLoad * kChunks),
                                       16, 0, 0);
#pragma unroll
    for (int i = 0; i < kBLoads; ++i)
      __builtin_amdgcn_global_load_lds(
          bp[i] + k0, (lds_ptr)(buf + (kWM + (w * kBLoads + i) * kRowsPerLoad) * kChunks), 16, 0, 0);
  };

  const int nk = K / kBK;
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st)
    if (st < nk) issue(st, st * kBK);
  for (int kt = 0; kt < nk; ++kt) {
    wait_ring<kStages - 2, kALoads + kBLoads>(nk - 1 - kt);
    ring_barrier();
    if (kt + kStages - 1 < nk) issue((kt + kStages - 1) % kStages, (kt + kStages - 1) * kBK);
    const u32x4* cur = lds[kt % kStages];
    const float s_gate = sw0[kt], s_up = sw1[kt];
    float sa[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) sa[t] = sap[t][kt];
    i32x8_t fb[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int row = kWM + wn * (kWT / 2) + 16 * t + r;
      fb[t] = cat8(cur[swz(row, 2 * q)], cur[swz(row, 2 * q + 1)]);
    }
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
      const int row = wm * (kWM / 2) + 16 * i + r;
      const i32x8_t fa = cat8(cur[swz(row, 2 * q)], cur[swz(row, 2 * q + 1)]);
      const float sw = (GATEUP && i >= kMT / 2) ? s_up : s_gate;
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        const f32x4 p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            fa, fb[t], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        acc[i][t] += p * (sw * sa[t]);
      }
    }
  }

  // Epilogue.
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int p = r0 + wn * (kWT / 2) + 16 * t + r;
    if (p >= n) continue;
    uint16_t* orow = dst + static_cast<int64_t>(row0 + p) * dst_ld;
    if (GATEUP) {
#pragma unroll
      for (int i = 0; i < kMT / 2; ++i) {
        float a[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) a[v] = silu(acc[i][t][v]) * acc[i + kMT / 2][t][v];
        const int ch = c0 + wm * (kWM / 4) + 16 * i + 4 * q;
        *reinterpret_cast<u32x2*>(orow + ch) = u32x2{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
      }
    } else {
#pragma unroll
      for (int i = 0; i < kMT; ++i) {
        const int h = c0 + wm * (kWM / 2) + 16 * i + 4 * q;
        *reinterpret_cast<u32x2*>(orow + h) =
            u32x2{pack_bf2(acc[i][t][0], acc[i][t][1]), pack_bf2(acc[i][t][2], acc[i][t][3])};
      }
    }
  }
}

}  // namespace f8t

hipError_t launch_gate_up_tiled_fp8(const GroupWeights& gw, const void* xq, const float* xs,
                                    const int32_t* counts, const int32_t* offsets,
                                    const int32_t* perm_tok, const int32_t* tiles, int max_tiles,
                                    int64_t T, int act_ld, void* act, hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  const int n_wtiles = Imax / (f8t::kWM / 2);
  f8t::tiled_fp8_kernel<true><<<round8(static_cast<int64_t>(max_tiles) * n_wtiles), 256, 0, s>>>(
      gw, static_cast<const uint8_t*>(xq), xs, gw.H, offsets, counts, perm_tok, tiles, max_tiles,
      n_wtiles, static_cast<int>(T), static_cast<uint16_t*>(act), act_ld);
  return hipGetLastError();
}

hipError_t launch_down_tiled_fp8(const GroupWeights& gw, const void* actq, const float* acts,
                                 int act_ld, const int32_t* counts, const int32_t* offsets,
                                 const int32_t* tiles, int max_tiles, int64_t T, void* out,
                                 hipStream_t s) {
  const int n_wtiles = gw.H / f8t::kWM;
  f8t::tiled_fp8_kernel<false><<<round8(static_cast<int64_t>(max_tiles) * n_wtiles), 256, 0, s>>>(
      gw, static_cast<const uint8_t*>(actq), acts, act_ld, offsets, counts, nullptr, tiles,
      max_tiles, n_wtiles, static_cast<int>(T), static_cast<uint16_t*>(out), gw.H);
  return hipGetLastError();
}

}  // namespace lbmoe
