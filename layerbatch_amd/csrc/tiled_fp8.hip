// LDS-tiled grouped GEMMs with fp8 (OCP e4m3) weights and activations, for prefill-sized
// batches: the products of the fp8 streaming kernels (fp8.hip) on the tile geometry, tile list,
// dispatch tables and global->LDS ring of the bf16 tiled GEMMs (tiled_shape.hpp,
// tiled_gemm.hip).
//
// A k-tile is 128 bytes per row = 128 e4m3 values = exactly one 128-k scale block, so it has
// the LDS geometry of a 64-value bf16 k-tile. One v_mfma_scale_f32_16x16x128_f8f6f4 covers a
// 16 x 16 output tile over the whole k-tile (lane (r, q) supplies bytes 32q .. 32q+31 of row
// r; OCP e4m3 operands, unit E8M0 scales). Its product p is scaled by
// w_scale(row block, k-tile) * a_scale(token, k-tile) and added to the fp32 accumulator; the
// fused multiply-adds of one MFMA step run under the next step's MFMAs.
// Workgroup: 8 waves in 2 x 4, kWM = 256 weight rows x 256 tokens (wide: a wave owns 128 rows
// x 64 tokens, 8 x 4 tiles of 16 x 16), x 128 tokens (narrow: 128 x 32) or, on 4 x 2 waves,
// x 64 tokens (tiny: 64 x 32). Accumulator lane (r, q) of a tile holds token column r and
// rows 4q .. 4q+3.
// Scales live in LDS for the whole work item: the activation scales of the tile's tokens for
// every k-tile (one 16-byte read per lane and k-tile) and the two weight-scale rows the
// workgroup's rows use; both are copied global -> LDS ahead of the ring's first stage.
#include "common.hpp"
#include "internal.hpp"
#include "offsets.hpp"
#include "tiled_shape.hpp"

namespace lbmoe {
namespace f8t {

// The LDS ring of 128-byte k-tiles (TileShape counts k-tiles in bf16 units: BK = 64).
using Wide = TileShape<2, 4, 2, 64, 2>;
using Narrow = TileShape<2, 4, 1, 64, 2>;
using Tiny = TileShape<4, 2, 1, 64, 3>;       // 4 x 2 waves of 64 x 32: 64 tokens
constexpr int kRingU4 = Wide::kStages * Wide::kStageU4;
static_assert(Narrow::kStages * Narrow::kStageU4 <= kRingU4, "narrow ring exceeds the wide one");
static_assert(Tiny::kStages * Tiny::kStageU4 <= kRingU4, "tiny ring exceeds the wide one");
// Scale blocks per row (K / 128) the LDS scale area holds: K <= 3072.
constexpr int kMaxKBlocks = 24;
constexpr int kActScales = kMaxKBlocks * Wide::kWT;
constexpr int kWScales = 64;                  // two rows of kMaxKBlocks, copied by one wave
static_assert(2 * kMaxKBlocks <= kWScales, "weight-scale rows exceed one wave copy");
static_assert(kRingU4 * 16 + (kActScales + kWScales) * 4 <= 160 * 1024, "LDS exceeds 160 KB");

__device__ __forceinline__ i32x8 cat8(u32x4 lo, u32x4 hi) {
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
               (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// Rows r0 .. r0 + S::kWT - 1 (clipped to n) of group g, output columns of weight tile wt.
// GATEUP: act[row, c] = silu(gate) * up over K = H, rounded to bf16 and quantised for the down
// GEMM: the tile's 128 channels are one quantisation group, so dst receives the e4m3 codes
// (dst_ld bytes per row) and dst_sc the group scales (dst_ld / 128 per row). Else out[row, h]
// (bf16, dst_ld per row) over K = Ig. row0: the group's first row in src (down) / dst. src_sc:
// per (row, 128 k) activation scales of src, src_ld / 128 per row.
// PERSIST: called from the persistent kernel's item loop, where the thread index goes through
// an empty asm, so the per-lane arithmetic is redone per item rather than hoisted out of the loop
// and held in registers across it.
template <bool GATEUP, class S, bool PERSIST = false>
__device__ __forceinline__ void tile_product_fp8(const GroupWeights& gw,
                                                 const uint8_t* __restrict__ src,
                                                 const float* __restrict__ src_sc, int src_ld,
                                                 const int32_t* __restrict__ perm_tok, int g,
                                                 int r0, int n, int row0, int wt,
                                                 void* __restrict__ dst, int dst_ld,
                                                 float* __restrict__ dst_sc,
                                                 u32x4* __restrict__ lds, float* __restrict__ scl) {
  constexpr int kM16 = 2 * S::kMT;               // 16-row tiles per wave
  constexpr int kN16 = 2 * S::kNT;               // 16-token tiles per wave
  constexpr int kRW = S::kRW, kWT = S::kWT, kWavesM = S::kWavesM;
  constexpr int kStages = S::kStages, kChunks = S::kChunks, kRowsPerLoad = S::kRowsPerLoad;
  constexpr int kALoads = S::kALoads, kBLoads = S::kBLoads, kLoads = S::kLoads;
  constexpr int kStageU4 = S::kStageU4;
  static_assert(kChunks == 8, "a k-tile is 128 bytes per row");
  const bool shared = g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int H = gw.H;
  const int K = GATEUP ? H : Ig;                 // bytes per weight row = k
  const int nk = K / 128;                        // k-tiles = scale blocks
  const int c0 = wt * (GATEUP ? kWM / 2 : kWM);  // first channel / output column

  int tid = threadIdx.x;
  if constexpr (PERSIST) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w % kWavesM, wn = w / kWavesM;

  // Weights and the two weight-scale rows (nk floats each) of the workgroup's rows. gate_up:
  // row 0 = the gate block of channels c0 .. c0+127, row 1 = their up block; down: the blocks
  // of output columns c0 .. c0+127 and c0+128 .. c0+255 (wave row-block wm uses row
  // wm * kRW / 128).
  const uint8_t* wbase;
  const uint8_t* wup = nullptr;
  const float* sw0;
  const float* sw1;
  if (GATEUP) {
    if (shared) {
      wbase = static_cast<const uint8_t*>(gw.sh_gate);
      wup = static_cast<const uint8_t*>(gw.sh_up);
      sw0 = gw.sh_gate_scale + static_cast<int64_t>(c0 / 128) * nk;
      sw1 = gw.sh_up_scale + static_cast<int64_t>(c0 / 128) * nk;
    } else {
      wbase = static_cast<const uint8_t*>(gw.gate_up) + static_cast<int64_t>(g) * 2 * gw.I * H;
      wup = wbase + static_cast<int64_t>(gw.I) * H;
      const float* s0 = gw.gate_up_scale + static_cast<int64_t>(g) * (2 * gw.I / 128) * nk;
      sw0 = s0 + static_cast<int64_t>(c0 / 128) * nk;
      sw1 = s0 + static_cast<int64_t>((gw.I + c0) / 128) * nk;
    }
  } else {
    if (shared) {
      wbase = static_cast<const uint8_t*>(gw.sh_down);
      sw0 = gw.sh_down_scale + static_cast<int64_t>(c0 / 128) * nk;
    } else {
      wbase = static_cast<const uint8_t*>(gw.down) + static_cast<int64_t>(g) * H * gw.I;
      sw0 = gw.down_scale + (static_cast<int64_t>(g) * (H / 128) + c0 / 128) * nk;
    }
    sw1 = sw0 + nk;
  }

  // Ring copies, as in the bf16 kernels: wave copy i fills one 1 KB LDS block of kRowsPerLoad
  // rows; lane l fetches the chunk that the swizzle places at slot l.
  const int lrow = lane / kChunks, lpos = lane % kChunks;
  // Copies through buffer resources, as in the bf16 kernels (there, global_load_lds made the
  // compiler wait for every outstanding LDS read before each MFMA step): a wave-uniform
  // descriptor per copy, a 32-bit lane offset (one VGPR per copy), the k-tile's byte step in
  // the scalar offset. The kRowsPerLoad rows of one copy are consecutive rows of one matrix.
  const uint8_t* abase[kALoads];
  uint32_t aoff[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int row0c = (w * kALoads + i) * kRowsPerLoad;        // the copy's first row
    const int row = row0c + lrow;
    const int j = lpos ^ ((row >> S::kSwzShift) & (kChunks - 1));
    if (GATEUP) {
      const int half = row0c / kRW, sub0 = row0c % kRW;
      abase[i] = sub0 < kRW / 2 ? wbase : wup;
      aoff[i] = static_cast<uint32_t>((c0 + half * (kRW / 2) + (sub0 % (kRW / 2)) + lrow) * K + 16 * j);
    } else {
      abase[i] = wbase;
      aoff[i] = static_cast<uint32_t>((c0 + row) * K + 16 * j);
    }
  }
  auto src_row = [&](int lt) {         // source row of local token lt (past n: a valid row)
    const int p = min(r0 + lt, n - 1);
    return GATEUP ? (shared ? p : perm_tok[row0 + p]) : row0 + p;
  };
  uint32_t boff[kBLoads];
#pragma unroll
  for (int i = 0; i < kBLoads; ++i) {
    const int lt = (w * kBLoads + i) * kRowsPerLoad + lrow;
    const int row = kWM + lt;
    const int j = lpos ^ ((row >> S::kSwzShift) & (kChunks - 1));
    boff[i] = static_cast<uint32_t>(src_row(lt)) * static_cast<uint32_t>(src_ld) + 16 * j;
  }

  typedef __attribute__((address_space(3))) void* lds_ptr;
  // Scale copies. Activation scales: token lt's row of nk scales goes to LDS as nc = ceil(nk/4)
  // 16-byte pieces, scl[lt * 4 nc + kb], a wave copy moving 64 pieces (64 / nc tokens' rows).
  // Copied as one 4-byte scale per lane (64 token rows per copy, each its own cache line) these
  // took 4x the copies and ~64 texture-address cycles apiece, ~4k cycles of every item's fill
  // at K = 2048. A row's last piece may reach 12 bytes past its nk scales (into the next row,
  // or the scale region's 16-byte tail). Wave 0 also copies the weight-scale rows.
  {
    const int nc = (nk + 3) / 4;
    const __amdgpu_buffer_rsrc_t srs = raw_rsrc(src_sc);
    const uint32_t row_bytes = static_cast<uint32_t>(src_ld / 128) * 4;
    for (int c0 = w * 64; c0 < kWT * nc; c0 += kThreads) {
      const int c = c0 + lane, lt = c / nc;
      const uint32_t off = static_cast<uint32_t>(src_row(lt)) * row_bytes + (c - lt * nc) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_ptr)(scl + c0 * 4), 16, off, 0, 0, 0);
    }
    if (w == 0) {
      const float* wsp = lane < nk ? sw0 + lane : (lane < 2 * nk ? sw1 + (lane - nk) : sw0);
      __builtin_amdgcn_global_load_lds(wsp, (lds_ptr)(scl + kActScales), 4, 0, 0);
    }
  }
  const float* wsc = scl + kActScales;

  f32x4 acc[kM16][kN16];
#pragma unroll
  for (int i = 0; i < kM16; ++i)
#pragma unroll
    for (int t = 0; t < kN16; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // narrow and tiny tiles' weight copies are non-temporal, as in the bf16 kernel
  constexpr int kWeightPolicy = S::kWT < kWM ? 2 : 0;
  __amdgpu_buffer_rsrc_t ars[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) ars[i] = raw_rsrc(abase[i]);
  const __amdgpu_buffer_rsrc_t brs = raw_rsrc(src);
  auto issue = [&](int stage, int k0) {
    u32x4* buf = lds + stage * kStageU4;
#pragma unroll
    for (int i = 0; i < kALoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ars[i], (lds_ptr)(buf + (w * kALoads + i) * kRowsPerLoad * kChunks), 16, aoff[i], k0,
          0, kWeightPolicy);
#pragma unroll
    for (int i = 0; i < kBLoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          brs, (lds_ptr)(buf + (kWM + (w * kBLoads + i) * kRowsPerLoad) * kChunks), 16, boff[i],
          k0, 0, 0);
  };

  const int r16 = lane & 15, q = lane >> 4;
  auto read_a = [&](const u32x4* buf, int i) {
    const int row = wm * kRW + 16 * i + r16;
    return cat8(buf[S::swz(row, 2 * q)], buf[S::swz(row, 2 * q + 1)]);
  };
  auto read_b = [&](const u32x4* buf, int t) {
    const int row = kWM + wn * (16 * kN16) + 16 * t + r16;
    return cat8(buf[S::swz(row, 2 * q)], buf[S::swz(row, 2 * q + 1)]);
  };
  // Ring protocol of the bf16 kernels: all kStages buffers are filled up front; in k-tile kt,
  // once the last A tile's fragments are in registers, each wave waits for its copies of
  // stage kt+1 and meets the others at the barrier, then reads stage kt+1's B fragments and
  // first A fragment and refills stage kt's buffer, interleaved with the last MFMAs.
  // a barrier after stage 0 puts every wave's stage 0 on the CU's copy path before any wave's
  // later stages (a wave reaches its wait only once it has issued all of its copies)
#pragma unroll
  for (int st = 0; st < kStages; ++st) {
    if (st < nk) issue(st, st * 128);
    if (st == 0) ring_barrier();
  }
  wait_ring<kStages - 1, kLoads>(nk - 1);
  ring_barrier();

  i32x8 fa[2], fb[kN16];
  f32x4 p[kN16];            // products of the previous MFMA step, not yet scaled and added
  float sp[kN16];           // their scales
#pragma unroll
  for (int t = 0; t < kN16; ++t) {
    fb[t] = read_b(lds, t);
    p[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    sp[t] = 0.f;
  }
  fa[0] = read_a(lds, 0);
  // Scales of k-tile kt: sc[h][t] = weight scale h * activation scale of column t, h = 0 for
  // gate and down tiles, 1 for up tiles. The next k-tile's are read at the k-tile's last step:
  // read halfway through, they held 6 more VGPRs over half of every k-tile (wide tiles 252 ->
  // 244 VGPRs, the same speed).
  float sa[kN16], w0, w1;
  const int scl_ld = 4 * ((nk + 3) / 4);          // activation scales per token in LDS
  auto read_scales = [&](int kt) {
    const float* a = scl + (wn * (16 * kN16) + r16) * scl_ld + kt;
#pragma unroll
    for (int t = 0; t < kN16; ++t) sa[t] = a[16 * t * scl_ld];
    w0 = wsc[(GATEUP ? 0 : wm * kRW / 128) * nk + kt];
    w1 = GATEUP ? wsc[nk + kt] : w0;
  };
  float sc[2][kN16];
  auto make_scales = [&]() {
#pragma unroll
    for (int t = 0; t < kN16; ++t) {
      sc[0][t] = w0 * sa[t];
      sc[1][t] = w1 * sa[t];
    }
  };
  read_scales(0);
  make_scales();

  // One step: the pending products are scaled and added just before the MFMA that replaces
  // them, one tile column at a time (VALU 4, MFMA 1), with the next A fragment's two reads
  // after the first MFMA.
  auto sched_step = [&]() {
#pragma unroll
    for (int t = 0; t < kN16; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (t == 0) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  auto ktile = [&]<bool NEXT, bool REFILL>(int kt) {
    const u32x4* cur = lds + (kt % kStages) * kStageU4;
#pragma unroll
    for (int i = 0; i < kM16; ++i) {
      const bool last = i == kM16 - 1;
      // the pending products belong to the previous step (at i = 0: the previous k-tile's
      // last step, or zeros with zero scales before the first k-tile)
      const int pi = i == 0 ? kM16 - 1 : i - 1;
      const int h = GATEUP && i >= kM16 / 2 ? 1 : 0;
      if (NEXT && i == kM16 - 1) read_scales(kt + 1);
      if (!last) fa[(i + 1) & 1] = read_a(cur, i + 1);
      if (last && NEXT) {
        // every earlier MFMA stays above the barrier
        __builtin_amdgcn_sched_barrier(0);
        wait_ring<kStages - 2, kLoads>(nk - 2 - kt);
        ring_barrier();
      }
      const u32x4* nxt = lds + ((kt + 1) % kStages) * kStageU4;
#pragma unroll
      for (int t = 0; t < kN16; ++t) {
        acc[pi][t] += p[t] * sp[t];
        p[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            fa[i & 1], fb[t], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        sp[t] = sc[h][t];
        if (last && NEXT) fb[t] = read_b(nxt, t);
      }
      if (last && NEXT) {
        fa[0] = read_a(nxt, 0);
        if constexpr (REFILL) issue(kt % kStages, (kt + kStages) * 128);
        make_scales();
        // next k-tile's B fragments one tile column at a time behind this step's MFMAs, then
        // its first A fragment and the refill copies
#pragma unroll
        for (int t = 0; t < kN16; ++t) {
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        if constexpr (REFILL) __builtin_amdgcn_sched_group_barrier(0x020, kLoads, 0);
      } else {
        sched_step();
      }
    }
  };
  int kt = 0;
  for (; kt + kStages < nk; ++kt) ktile.template operator()<true, true>(kt);
  for (; kt + 1 < nk; ++kt) ktile.template operator()<true, false>(kt);
  ktile.template operator()<false, false>(kt);
#pragma unroll
  for (int t = 0; t < kN16; ++t) acc[kM16 - 1][t] += p[t] * sp[t];

  // Epilogue: stage the tile in the ring as [token][column] bf16, then store row segments.
  constexpr int kCols = GATEUP ? kWM / 2 : kWM;
  static_assert(kWT * (kCols / 8) <= kRingU4, "staged tile exceeds the LDS ring");
  ring_barrier();                                           // every wave is done with the ring
  char* st = reinterpret_cast<char*>(lds);
#pragma unroll
  for (int t = 0; t < kN16; ++t) {
    const int r = wn * (16 * kN16) + 16 * t + r16;          // token within the tile
#pragma unroll
    for (int i = 0; i < (GATEUP ? kM16 / 2 : kM16); ++i) {
      float a[4];
#pragma unroll
      for (int v = 0; v < 4; ++v)
        a[v] = GATEUP ? silu(acc[i][t][v]) * acc[i + kM16 / 2][t][v] : acc[i][t][v];
      const int c = (GATEUP ? wm * (kRW / 2) : wm * kRW) + 16 * i + 4 * q;
      *reinterpret_cast<u32x2*>(st + staged_slot<kCols>(r, c / 8) * 16 + (c % 8) * 2) =
          u32x2{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
    }
  }
  ring_barrier();
  if constexpr (GATEUP) {
    // 16 lanes per token: the group's amax, scale and codes (as quant_groups_kernel computes
    // them from the stored bf16 act). All of a thread's tokens at once, so that their
    // independent chains (LDS read, row maximum, divisions) overlap; tokens past the group's
    // rows are computed from whatever the staging area holds and not stored.
    uint8_t* q = static_cast<uint8_t*>(dst);
    const int sub = tid & 15;
    constexpr int kPer = kThreads / 16, kIters = kWT / kPer;
    static_assert(kWT % kPer == 0, "tokens per pass divide the tile");
    u32x4 v[kIters];
#pragma unroll
    for (int i = 0; i < kIters; ++i) v[i] = lds[staged_slot<kCols>((tid >> 4) + i * kPer, sub)];
#pragma unroll
    for (int i = 0; i < kIters; ++i) {
      const int p = r0 + (tid >> 4) + i * kPer;
      float sc;
      const u32x2 c = quant_group16(v[i], sc);
      if (p < n) {
        const int64_t row = row0 + p;
        *reinterpret_cast<u32x2*>(q + row * dst_ld + c0 + 8 * sub) = c;
        if (sub == 0) dst_sc[row * (dst_ld / 128) + c0 / 128] = sc;
      }
    }
  } else {
    store_staged<kCols, kWT, true>(lds, static_cast<uint16_t*>(dst), dst_ld, row0, r0, n, c0);
  }
}

template <bool GATEUP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tiled_fp8_kernel(GroupWeights gw, const uint8_t* __restrict__ src,
                      const float* __restrict__ src_sc, int src_ld,
                      const int32_t* __restrict__ perm_tok, const u32x4* __restrict__ table,
                      void* __restrict__ dst, int dst_ld, float* __restrict__ dst_sc) {
  __shared__ u32x4 lds[kRingU4];
  __shared__ float scl[kActScales + kWScales];
  const TileItem it = decode_item(table[blockIdx.x]);
  if (it.g < 0) return;
  if (it.tiny)
    tile_product_fp8<GATEUP, Tiny>(gw, src, src_sc, src_ld, perm_tok, it.g, it.r0, it.n,
                                   it.row0, it.wt, dst, dst_ld, dst_sc, lds, scl);
  else if (it.narrow)
    tile_product_fp8<GATEUP, Narrow>(gw, src, src_sc, src_ld, perm_tok, it.g, it.r0, it.n,
                                     it.row0, it.wt, dst, dst_ld, dst_sc, lds, scl);
  else
    tile_product_fp8<GATEUP, Wide>(gw, src, src_sc, src_ld, perm_tok, it.g, it.r0, it.n,
                                   it.row0, it.wt, dst, dst_ld, dst_sc, lds, scl);
}

// gate_up as one workgroup per CU taking entries from the per-XCD work queues of the dispatch
// table (queue_fetch): thread 0 claims the next entry once the previous item's stores have gone
// out, and the barrier after it also orders the item's staging reads before the next fill.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tiled_fp8_persistent_kernel(GroupWeights gw, const uint8_t* __restrict__ src,
                                 const float* __restrict__ src_sc, int src_ld,
                                 const int32_t* __restrict__ perm_tok,
                                 const u32x4* __restrict__ table, int slots, int* __restrict__ q,
                                 void* __restrict__ dst, int dst_ld, float* __restrict__ dst_sc) {
  __shared__ u32x4 lds[kRingU4];
  __shared__ float scl[kActScales + kWScales];
  __shared__ u32x4 ent;
  __shared__ int tried;                // the queue state lives in LDS, not across the loop
  if (threadIdx.x == 0) tried = 0;
  for (;;) {
    if (threadIdx.x == 0) {
      WorkQueue wq{table, slots, q, static_cast<int>(blockIdx.x & 7), tried, 0};
      ent = queue_fetch(wq);
      tried = wq.tried;
    }
    __syncthreads();
    const TileItem it = decode_item(ent);
    if (it.g < 0) break;               // the same for the whole workgroup
    if (it.tiny)
      tile_product_fp8<true, Tiny, true>(gw, src, src_sc, src_ld, perm_tok, it.g, it.r0, it.n,
                                         it.row0, it.wt, dst, dst_ld, dst_sc, lds, scl);
    else if (it.narrow)
      tile_product_fp8<true, Narrow, true>(gw, src, src_sc, src_ld, perm_tok, it.g, it.r0, it.n,
                                           it.row0, it.wt, dst, dst_ld, dst_sc, lds, scl);
    else
      tile_product_fp8<true, Wide, true>(gw, src, src_sc, src_ld, perm_tok, it.g, it.r0, it.n,
                                         it.row0, it.wt, dst, dst_ld, dst_sc, lds, scl);
  }
}

}  // namespace f8t

bool tiled_fp8_supported(const GroupWeights& gw, int64_t T, int64_t rows) {
  // the copies address operands with byte offsets below 2^31 from a weight matrix, xq or actq
  return tiled_supported(gw) && gw.H / 128 <= f8t::kMaxKBlocks &&
         gw.I / 128 <= f8t::kMaxKBlocks && gw.Is / 128 <= f8t::kMaxKBlocks &&
         fp8_tiled_offsets_fit(T, rows, gw.H, gw.I > gw.Is ? gw.I : gw.Is);
}

hipError_t launch_gate_up_tiled_fp8(const GroupWeights& gw, const void* xq, const float* xs,
                                    const int32_t* perm_tok, const int32_t* tiles, int max_tiles,
                                    int act_ld, void* actq, float* acts, hipStream_t s) {
  const int grid = tiled_grid(gw, max_tiles, true), cus = device_cus();
  const u32x4* table = tiled_table(gw, tiles, max_tiles, true);
  if (grid >= kPersistentMinEntriesPerCu * cus) {
    int32_t* q = queue_base(const_cast<int32_t*>(tiles), max_tiles, grid,
                            tiled_grid(gw, max_tiles, false));
    f8t::tiled_fp8_persistent_kernel<<<cus, kThreads, 0, s>>>(
        gw, static_cast<const uint8_t*>(xq), xs, gw.H, perm_tok, table, grid / 8, q, actq, act_ld,
        acts);
  } else {
    f8t::tiled_fp8_kernel<true><<<grid, kThreads, 0, s>>>(
        gw, static_cast<const uint8_t*>(xq), xs, gw.H, perm_tok, table, actq, act_ld, acts);
  }
  return hipGetLastError();
}

hipError_t launch_down_tiled_fp8(const GroupWeights& gw, const void* actq, const float* acts,
                                 int act_ld, const int32_t* tiles, int max_tiles, void* out,
                                 hipStream_t s) {
  f8t::tiled_fp8_kernel<false><<<tiled_grid(gw, max_tiles, false), kThreads, 0, s>>>(
      gw, static_cast<const uint8_t*>(actq), acts, act_ld, nullptr,
      tiled_table(gw, tiles, max_tiles, false), out, gw.H, nullptr);
  return hipGetLastError();
}

}  // namespace lbmoe
