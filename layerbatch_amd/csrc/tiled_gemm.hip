// LDS-tiled grouped GEMMs for prefill-sized batches (gfx950, v_mfma_f32_32x32x16_bf16).
//
// Same products as the streaming kernels (gate_up + SiLU*mul, qwen3_5.py:835-836; down,
// qwen3_5.py:837), for groups with many tokens: a workgroup multiplies a tile of kWM weight
// rows by a tile of kWT tokens of one expert, staging both operands through LDS in k-tiles of
// kBK, so each operand byte fetched from L2 feeds kWT (or kWM) MFMA columns. The k-tiles move
// global -> LDS directly (global_load_lds_dwordx4, no register staging) through a ring of
// kStages buffers, loads running kStages-1 tiles ahead of the MFMAs.
//
// Work list. build_tiles turns the per-expert token counts into a list of (group, first row)
// token tiles; a launch covers max_tiles x n_tiles workgroups (a function of T only) and
// workgroups past the list's end exit. Consecutive workgroups of one XCD take consecutive
// (token tile, weight tile) pairs, weight tile fastest, so the tiles that share a token tile
// run together on one XCD's L2.
//
// Layout. A = weight rows (MFMA rows), B = tokens (MFMA columns). Accumulator lane l of a
// 32x32 tile holds token column l%32 and weight rows 8(v/4) + 4(l/32) + v%4, v = 0..15, so
// four consecutive output channels of one token are stored together. LDS rows are kBK bf16
// (64 bytes) in 16-byte chunks; chunk j of row r is stored at chunk j ^ ((r >> 2) & 3), which
// keeps the 32-row MFMA operand reads free of bank conflicts.
// Gate_up workgroups take kWM/2 channels: wave row-half h holds gate rows then up rows of the
// same kWM/4 channels, so SiLU*mul pairs accumulators in registers.
#include "common.hpp"
#include "internal.hpp"
#include "tiled_common.hpp"

namespace lbmoe {

// Tile configuration: kWavesM x kWavesN waves per workgroup, each wave owning kMT x kNT
// 32x32 MFMA tiles (weights x tokens).
#ifndef LBMOE_TILE_WAVES_N
#define LBMOE_TILE_WAVES_N 1
#endif
#ifndef LBMOE_TILE_NT
#define LBMOE_TILE_NT 4
#endif
#ifndef LBMOE_TILE_WPE
#define LBMOE_TILE_WPE 1
#endif
constexpr int kWavesM = 2;
constexpr int kWavesN = LBMOE_TILE_WAVES_N;
constexpr int kMT = 4;                              // 32-row MFMA tiles per wave (weights)
constexpr int kNT = LBMOE_TILE_NT;                  // 32-column MFMA tiles per wave (tokens)
constexpr int kWaves = kWavesM * kWavesN;
constexpr int kThreads = 64 * kWaves;
constexpr int kWM = kWavesM * kMT * 32;             // weight rows per workgroup
constexpr int kWT = kWavesN * kNT * 32;             // tokens per workgroup
#ifndef LBMOE_TILE_BK
#define LBMOE_TILE_BK 32
#endif
constexpr int kBK = LBMOE_TILE_BK;                  // k per LDS stage
#ifndef LBMOE_TILE_STAGES
#define LBMOE_TILE_STAGES 3
#endif
constexpr int kStages = LBMOE_TILE_STAGES;          // LDS ring depth
constexpr int kChunks = kBK / 8;                    // 16-byte chunks per LDS row
constexpr int kRowsPerLoad = 64 / kChunks;          // rows one wave load covers
constexpr int kALoads = kWM / kRowsPerLoad / kWaves;   // wave loads per stage (weights)
constexpr int kBLoads = kWT / kRowsPerLoad / kWaves;   // wave loads per stage (tokens)
constexpr int kStageU4 = (kWM + kWT) * kChunks;     // 16-byte slots per stage
static_assert(kALoads * kRowsPerLoad * kWaves == kWM && kBLoads * kRowsPerLoad * kWaves == kWT,
              "loads must tile the stage");

constexpr int kKSteps = kBK / 16;                  // MFMA k-steps per stage
// Chunk j of LDS row r lives at slot r*kChunks + (j ^ f(r)), f(r) = (r / (16/kChunks)) mod
// kChunks: 16 consecutive rows then hit 16 distinct 16-byte bank groups for any fixed j.
constexpr int kSwzShift = kChunks == 4 ? 2 : 1;
static_assert(kChunks == 4 || kChunks == 8, "kBK must be 32 or 64");
__device__ __forceinline__ int swz(int r, int j) {
  return r * kChunks + (j ^ ((r >> kSwzShift) & (kChunks - 1)));
}

// ---- tile list -------------------------------------------------------------------------------
// tiles[2i] = group, tiles[2i+1] = first row within the group, in group order;
// tiles[2*max_tiles] = number of valid entries. Groups: routed experts 0..E-1 with counts[g]
// rows, then the shared expert (T rows) when present.
__global__ __launch_bounds__(1024) void build_tiles_kernel(const int32_t* __restrict__ counts,
                                                           int E, int shared, int T, int max_tiles,
                                                           int32_t* __restrict__ tiles) {
  __shared__ int wsum[16];
  const int G = E + shared;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (G + 1023) / 1024;
  const int lo = min(G, tid * per), hi = min(G, lo + per);
  int local = 0;
  for (int g = lo; g < hi; ++g) {
    const int n = g < E ? counts[g] : T;
    local += (n + kWT - 1) / kWT;
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < 16 ? wsum[lane] : 0;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(w, o, kWave);
      if (lane >= o) w += y;
    }
    if (lane < 16) wsum[lane] = w;
  }
  __syncthreads();
  int pos = incl - local + (wave > 0 ? wsum[wave - 1] : 0);
  for (int g = lo; g < hi; ++g) {
    const int n = g < E ? counts[g] : T;
    for (int r = 0; r < n; r += kWT) {
      if (pos < max_tiles) {
        tiles[2 * pos] = g;
        tiles[2 * pos + 1] = r;
      }
      ++pos;
    }
  }
  if (tid == 0) tiles[2 * max_tiles] = min(wsum[15], max_tiles);
}

// ---- the tiled kernel ----------------------------------------------------------------------
// MODE kDown: out[row, h] = act[row] . Wd_g[h];  kGateUp: act[row, c] = silu(gate) * up;
// kRouter: logits[t, e] = x[t] . Wg[e] over token tiles t0 = 128 * tile (no tile list;
// gw.gate_up holds the router weight, gw.E its row count).
enum TileMode { kDown = 0, kGateUp = 1, kRouter = 2 };

template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(LBMOE_TILE_WPE, LBMOE_TILE_WPE))) void tiled_kernel(GroupWeights gw, const uint16_t* __restrict__ src,
                                                    int src_ld, const int32_t* __restrict__ offsets,
                                                    const int32_t* __restrict__ counts,
                                                    const int32_t* __restrict__ perm_tok,
                                                    const int32_t* __restrict__ tiles,
                                                    int max_tiles, int n_wtiles, int T,
                                                    uint16_t* __restrict__ dst, int dst_ld) {
  constexpr bool GATEUP = MODE == kGateUp, ROUTER = MODE == kRouter;
  __shared__ u32x4 lds[kStages][kStageU4];
  // XCD-aware order: hardware hands out workgroup b to XCD b % 8.
  const int logical = xcd_logical_block(blockIdx.x, gridDim.x);
  const int ti = logical / n_wtiles, wt = logical - ti * n_wtiles;
  int g = 0, r0, n, row0;
  if (ROUTER) {
    if (ti * kWT >= T) return;
    r0 = ti * kWT;
    n = T;
    row0 = 0;
  } else {
    if (ti >= tiles[2 * max_tiles]) return;
    g = tiles[2 * ti];
    r0 = tiles[2 * ti + 1];
  }
  const bool shared = !ROUTER && g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int H = gw.H;
  if (!ROUTER) {
    n = shared ? T : counts[g];
    row0 = shared ? gw.sh_row0 : offsets[g];
  }
  const int K = (GATEUP || ROUTER) ? H : Ig;
  const int c0 = wt * (GATEUP ? kWM / 2 : kWM);      // first channel / output column
  if (c0 >= (GATEUP ? Ig : (ROUTER ? gw.E : H))) return;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w % kWavesM, wn = w / kWavesM;

  // Direct global->LDS loads: wave load i writes one contiguous 1 KB LDS block of
  // kRowsPerLoad rows; lane l fills slot l of it, i.e. row R0 + l/kChunks at swizzled position
  // l%kChunks, so it fetches the chunk that the swizzle places there.
  const uint16_t* wbase;
  const uint16_t* wup = nullptr;
  if (GATEUP) {
    if (shared) {
      wbase = static_cast<const uint16_t*>(gw.sh_gate);
      wup = static_cast<const uint16_t*>(gw.sh_up);
    } else {
      wbase = static_cast<const uint16_t*>(gw.gate_up) + static_cast<int64_t>(g) * 2 * gw.I * H;
      wup = wbase + static_cast<int64_t>(gw.I) * H;
    }
  } else if (ROUTER) {
    wbase = static_cast<const uint16_t*>(gw.gate_up);
  } else {
    wbase = shared ? static_cast<const uint16_t*>(gw.sh_down)
                   : static_cast<const uint16_t*>(gw.down) + static_cast<int64_t>(g) * H * gw.I;
  }
  const int lrow = lane / kChunks, lpos = lane % kChunks;
  const uint16_t* ap[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int row = (w * kALoads + i) * kRowsPerLoad + lrow;    // local weight row
    const int j = lpos ^ ((row >> kSwzShift) & (kChunks - 1));
    int grow;
    const uint16_t* base = wbase;
    if (GATEUP) {
      const int half = row / (kWM / 2), sub = row % (kWM / 2);
      base = sub < kWM / 4 ? wbase : wup;
      grow = c0 + half * (kWM / 4) + (sub % (kWM / 4));
    } else if (ROUTER) {
      grow = min(c0 + row, gw.E - 1);      // rows past E repeat a valid row; not stored
    } else {
      grow = c0 + row;
    }
    ap[i] = base + static_cast<int64_t>(grow) * K + 8 * j;
  }
  const uint16_t* bp[kBLoads];
#pragma unroll
  for (int i = 0; i < kBLoads; ++i) {
    const int lt = (w * kBLoads + i) * kRowsPerLoad + lrow;     // local token
    const int row = kWM + lt;
    const int j = lpos ^ ((row >> kSwzShift) & (kChunks - 1));
    const int p = min(r0 + lt, n - 1);   // rows past the group repeat a valid row; not stored
    const int srow = ROUTER ? p : (GATEUP ? (shared ? p : perm_tok[row0 + p]) : row0 + p);
    bp[i] = src + static_cast<int64_t>(srow) * src_ld + 8 * j;
  }

  f32x16 acc[kMT][kNT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

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
      __builtin_amdgcn_global_load_lds(bp[i] + k0,
                                       (lds_ptr)(buf + (kWM + (w * kBLoads + i) * kRowsPerLoad) * kChunks),
                                       16, 0, 0);
  };

  const int nk = K / kBK;
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st)
    if (st < nk) issue(st, st * kBK);
  const int mr = lane & 31, mk = lane >> 5;   // MFMA operand: row l%32, k-chunk half l/32
  auto read_frags = [&](const u32x4* cur, int ks, u32x4 (&fa)[kMT], u32x4 (&fb)[kNT]) {
    const int j = 2 * ks + mk;
#pragma unroll
    for (int i = 0; i < kMT; ++i) fa[i] = cur[swz(wm * (kWM / 2) + 32 * i + mr, j)];
#pragma unroll
    for (int t = 0; t < kNT; ++t) fb[t] = cur[swz(kWM + wn * (kNT * 32) + 32 * t + mr, j)];
  };
  for (int kt = 0; kt < nk; ++kt) {
    wait_ring<kStages - 2, kALoads + kBLoads>(nk - 1 - kt);
    ring_barrier();
    if (kt + kStages - 1 < nk) issue((kt + kStages - 1) % kStages, (kt + kStages - 1) * kBK);
    const u32x4* cur = lds[kt % kStages];
    u32x4 fa[2][kMT], fb[2][kNT];
    read_frags(cur, 0, fa[0], fb[0]);
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      if (ks + 1 < kKSteps) read_frags(cur, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(fa[ks & 1][i]),
                                                              as_bf16x8(fb[ks & 1][t]),
                                                              acc[i][t], 0, 0, 0);
    }
    // Schedule: the first k-step's fragment reads, then each later k-step's reads
    // interleaved one-for-one with the previous k-step's MFMAs.
    __builtin_amdgcn_sched_group_barrier(0x100, kMT + kNT, 0);
#pragma unroll
    for (int ks = 0; ks + 1 < kKSteps; ++ks) {
#pragma unroll
      for (int r = 0; r < kMT + kNT; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kMT * kNT - (kMT + kNT), 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kMT * kNT, 0);
  }

  // Epilogue.
  const int col = lane & 31, rq = 4 * (lane >> 5);
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int p = r0 + wn * (kNT * 32) + 32 * t + col;
    if (p >= n) continue;
    uint16_t* orow = dst + static_cast<int64_t>(row0 + p) * dst_ld;
    if (GATEUP) {
#pragma unroll
      for (int i = 0; i < kMT / 2; ++i)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          float a[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            a[v] = silu(acc[i][t][4 * v4 + v]) * acc[i + kMT / 2][t][4 * v4 + v];
          const int ch = c0 + wm * (kWM / 4) + 32 * i + 8 * v4 + rq;
          *reinterpret_cast<u32x2*>(orow + ch) = u32x2{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
        }
    } else if (ROUTER) {
      const int E = gw.E;
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const int e = c0 + wm * (kWM / 2) + 32 * i + 8 * v4 + rq;
          if (e + 3 < E && (E & 3) == 0) {
            *reinterpret_cast<u32x2*>(orow + e) =
                u32x2{pack_bf2(acc[i][t][4 * v4], acc[i][t][4 * v4 + 1]),
                      pack_bf2(acc[i][t][4 * v4 + 2], acc[i][t][4 * v4 + 3])};
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (e + v < E) orow[e + v] = static_cast<uint16_t>(f2bf(acc[i][t][4 * v4 + v]));
          }
        }
    } else {
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const int h = c0 + wm * (kWM / 2) + 32 * i + 8 * v4 + rq;
          *reinterpret_cast<u32x2*>(orow + h) =
              u32x2{pack_bf2(acc[i][t][4 * v4], acc[i][t][4 * v4 + 1]),
                    pack_bf2(acc[i][t][4 * v4 + 2], acc[i][t][4 * v4 + 3])};
        }
    }
  }
}

// Upper bound of the token-tile count: every group adds at most one partial tile.
int tiled_max_tiles(int64_t rows, int groups) {
  return static_cast<int>((rows + kWT - 1) / kWT) + groups + 1;
}

bool tiled_supported(const GroupWeights& gw) {
  return gw.H % kWM == 0 && gw.H % kBK == 0 && gw.I % (kWM / 2) == 0 &&
         (gw.Is == 0 || gw.Is % (kWM / 2) == 0) && gw.I % kBK == 0 && gw.I < (1 << 20);
}

hipError_t launch_build_tiles(const int32_t* counts, int E, bool shared, int64_t T, int max_tiles,
                              int32_t* tiles, hipStream_t s) {
  build_tiles_kernel<<<1, 1024, 0, s>>>(counts, E, shared ? 1 : 0, static_cast<int>(T), max_tiles,
                                        tiles);
  return hipGetLastError();
}


hipError_t launch_gate_up_tiled(const GroupWeights& gw, const void* x, const int32_t* counts,
                                const int32_t* offsets, const int32_t* perm_tok,
                                const int32_t* tiles, int max_tiles, int64_t T, int act_ld,
                                void* act, hipStream_t s) {
  const int Imax = gw.I > gw.Is ? gw.I : gw.Is;
  const int n_wtiles = Imax / (kWM / 2);
  tiled_kernel<kGateUp><<<round8(static_cast<int64_t>(max_tiles) * n_wtiles), kThreads, 0, s>>>(
      gw, static_cast<const uint16_t*>(x), gw.H, offsets, counts, perm_tok, tiles, max_tiles,
      n_wtiles, static_cast<int>(T), static_cast<uint16_t*>(act), act_ld);
  return hipGetLastError();
}

hipError_t launch_down_tiled(const GroupWeights& gw, const void* act, int act_ld,
                             const int32_t* counts, const int32_t* offsets, const int32_t* tiles,
                             int max_tiles, int64_t T, void* out, hipStream_t s) {
  const int n_wtiles = gw.H / kWM;
  tiled_kernel<kDown><<<round8(static_cast<int64_t>(max_tiles) * n_wtiles), kThreads, 0, s>>>(
      gw, static_cast<const uint16_t*>(act), act_ld, offsets, counts, nullptr, tiles, max_tiles,
      n_wtiles, static_cast<int>(T), static_cast<uint16_t*>(out), gw.H);
  return hipGetLastError();
}

}  // namespace lbmoe

namespace lbmoe {

bool tiled_router_supported(int E, int H) { return H % kBK == 0 && E >= 1; }

hipError_t launch_router_logits_tiled(const void* x, const void* wg, int64_t T, int E, int H,
                                      void* logits, hipStream_t s) {
  GroupWeights gw{};
  gw.gate_up = wg;
  gw.E = E;
  gw.H = H;
  const int n_wtiles = (E + kWM - 1) / kWM;
  const int64_t n_ttiles = (T + kWT - 1) / kWT;
  tiled_kernel<kRouter><<<round8(n_ttiles * n_wtiles), kThreads, 0, s>>>(
      gw, static_cast<const uint16_t*>(x), H, nullptr, nullptr, nullptr, nullptr, 0, n_wtiles,
      static_cast<int>(T), static_cast<uint16_t*>(logits), E);
  return hipGetLastError();
}

}  // namespace lbmoe
