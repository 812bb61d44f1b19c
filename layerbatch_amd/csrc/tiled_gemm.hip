// LDS-tiled grouped GEMMs for prefill-sized batches (gfx950, v_mfma_f32_32x32x16_bf16).
//
// Same products as the streaming kernels (gate_up + SiLU*mul, qwen3_5.py:835-836; down,
// qwen3_5.py:837), for groups with many tokens: a workgroup of 8 waves (two per SIMD, so one
// wave's copy issue and LDS waits overlap the other's MFMAs) multiplies a tile of kWM = 256
// weight rows by a tile of tokens of one expert, staging both operands
// through LDS in k-tiles, so each operand byte fetched from L2 feeds many MFMA columns. The
// k-tiles move global -> LDS directly (global_load_lds_dwordx4, no register staging) through
// a ring of LDS buffers that is filled kStages k-tiles ahead of the MFMAs. The wide tiles'
// weight operand has one stage more than its token operand (3 + 2 stages of 32 KB, the CU's
// whole 160 KB): the weight copies, which may stream from HBM, get a k-tile longer to land.
//
// Two token-tile widths share one launch. A wide tile (256 tokens, each wave 128 x 64) moves
// the fewest operand bytes per flop, which matters here: with the whole chip busy the shader
// clock settles near 1.5 GHz and every byte moved between L2 and LDS costs cycles and power.
// A narrow tile (128 tokens, each wave 128 x 32) serves the few tokens that small experts get
// under a skewed router: such a tile is bound by streaming the expert's weights from HBM, and
// a wide tile would spend twice the MFMA work on padding. A tiny tile (64 tokens, each wave
// 64 x 32) takes a group's last rows when there are at most 64 of them, which under a skewed
// router is most experts. Because the tile list follows expert order, narrow and tiny
// (HBM-bound) and wide (MFMA-bound) tiles run side by side.
//
// Work list. build_tiles turns the per-expert token counts into a list of (group, first row |
// narrow or tiny flag) token tiles, wide ones first; a launch has one workgroup per possible
// (token tile, weight tile) item (a function of T only), and dispatch_item maps workgroups to
// items so that each XCD works on its own share, with small-expert tiles spread over the
// launch and its last round.
//
// Layout. A = weight rows (MFMA rows), B = tokens (MFMA columns). Accumulator lane l of a
// 32x32 tile holds token column l%32 and weight rows 8(v/4) + 4(l/32) + v%4, v = 0..15, so
// four consecutive output channels of one token are stored together. LDS rows are kBK bf16 in
// 16-byte chunks; chunk j of row r is stored at a row-dependent XOR of j (swz), which keeps
// the 32-row MFMA operand reads free of bank conflicts.
// Gate_up workgroups take kWM/2 channels: the weight rows alternate in 32-row blocks between
// the gate and the up rows of the same 32 channels, so SiLU*mul pairs accumulators in registers.
//
// Weights come either in the checkpoint layout ([E,2I,H], [E,H,I]) or, when the caller has
// packed them (lbmoe_pack_weights -> pack_tiled_kernel), in a tiled layout where each k-tile of
// a weight tile is one contiguous 32 KB block already in LDS order. HBM streams those blocks
// markedly faster than 256 row segments of 128 bytes spread over 1 MB (a read probe in the
// ring's pattern, with token copies that hit L2 as here: 6.7 against 5.2 TB/s).
#include <atomic>

#include "common.hpp"
#include "internal.hpp"
#include "offsets.hpp"
#include "route_token.hpp"
#include "tiled_shape.hpp"

namespace lbmoe {

// wide: 2 x 4 waves of 128 x 64 (256 tokens), 3 weight + 2 token stages of 64-k tiles; narrow:
// 4 x 2 waves of 64 x 64 (128 tokens; four fragment reads per k-step instead of the five of
// 2 x 4 waves of 128 x 32: E=512 T=4096 gate_up 396 -> 390 us, layer 710.6 -> 707.4 us
// median), 3 stages of both
using Wide = TileShape<2, 4, 2, 64, 3, 2>;
using Narrow = TileShape<4, 2, 2, 64, 3>;
// tiny: 4 x 2 waves of 64 x 32 (64 tokens), for a group's last few rows
using Tiny = TileShape<4, 2, 1, 64, 3>;
// router logits: 4 x 2 waves of 64 x 32 (256 experts x 64 tokens); for at most 128 experts
// 4 x 2 waves of 32 x 32 (128 x 64) with a ring small enough for two workgroups per CU
using RouterShape = TileShape<4, 2, 1, 64, 3>;
using RouterShape128 = TileShape<4, 1, 1, 64, 3>;
// for batches that fill the chip with it: 2 x 4 waves of 128 x 32 (256 experts x 128 tokens),
// which moves fewer operand bytes per flop than 64-token tiles
using RouterShapeTall = TileShape<2, 4, 1, 64, 3>;
constexpr int64_t kRouterTallMinWorkgroups = 256;
constexpr int kLdsU4 = Wide::kRingU4 > Narrow::kRingU4 ? Wide::kRingU4 : Narrow::kRingU4;
static_assert(Tiny::kRingU4 <= kLdsU4, "tiny ring exceeds the others");
static_assert(kLdsU4 * 16 <= 160 * 1024, "LDS ring exceeds the CU's 160 KB");

// ---- tile list -------------------------------------------------------------------------------
// tiles[2i] = group, tiles[2i+1] = first row within the group (| kNarrowFlag for a narrow
// tile, | kTinyFlag for a tiny one). All wide tiles come first, in group order, then all
// narrow and tiny tiles, in group order.
// Behind the max_tiles entries: tiles[2*max_tiles] = number of valid entries,
// tiles[2*max_tiles+1] = number of wide entries. Groups: routed experts 0..E-1 with counts[g]
// rows, then the shared expert (T rows) when present. A group of n rows gets n / wide wide
// tiles; the remainder r is one more wide tile when r > wide - narrow (or when narrow == 0),
// else one tiny tile when r <= tiny, else ceil(r / narrow) narrow tiles.
__device__ __forceinline__ void group_tiles(int n, int wide, int narrow, int tiny, int& n_wide,
                                            int& n_narrow, int& n_tiny) {
  n_wide = n / wide;
  n_narrow = 0;
  n_tiny = 0;
  const int r = n - n_wide * wide;
  if (r == 0) return;
  if (narrow == 0 || r > wide - narrow) ++n_wide;
  else if (r <= tiny) n_tiny = 1;
  else n_narrow = (r + narrow - 1) / narrow;
}

// Block-wide exclusive scan of one int per thread (1024 threads); returns the total.
__device__ __forceinline__ int block_scan_1024(int v, int& excl, int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    const int c = wsum[w];
    before += w < wave ? c : 0;
    total += c;
  }
  excl = before + incl - v;
  __syncthreads();
  return total;
}

// Dispatch order of the GEMM items. Items are (token tile, weight tile) pairs, weight tile
// fastest; the W wide items come first, then the N narrow and tiny ones (both "narrow" below).
// XCD x owns the x-th contiguous eighth of the wide items and of the narrow items, so items
// that share a token tile run on one L2. Within an XCD the hardware hands out workgroups in
// order as CUs free up, so slot j (= blockIdx / 8) is roughly a point in time: the XCD's last
// kTailSlots slots go to narrow (short, HBM-bound) items, so that the launch ends on short
// items, and its other narrow items are spread evenly between the wide (MFMA-bound) ones, so
// that weight streaming for small experts overlaps MFMA work. Returns the item of workgroup b,
// or -1.
constexpr int kTailSlots = 32;
__device__ __forceinline__ int dispatch_item(int b, int W, int N) {
  const int x = b & 7, j = b >> 3;
  const int cw = (W + 7) >> 3, cn = (N + 7) >> 3;
  const int w0 = min(W, x * cw), nw = min(W, w0 + cw) - w0;     // this XCD's wide items
  const int n0 = min(N, x * cn), nn = min(N, n0 + cn) - n0;     // and narrow items
  if (j >= nw + nn) return -1;
  const int tail = min(nn, kTailSlots);
  const int spread = nn - tail, prefix = nw + spread;
  if (j >= prefix) return W + n0 + spread + (j - prefix);       // the tail: narrow items
  // narrow items before slot j in the prefix: floor(j * spread / prefix)
  const int before = static_cast<int>(static_cast<int64_t>(j) * spread / prefix);
  const int upto = static_cast<int>(static_cast<int64_t>(j + 1) * spread / prefix);
  return upto > before ? W + n0 + before : w0 + (j - before);
}


// One entry of a dispatch table: the work of workgroup b of a bf16 GEMM launch, read with a
// single 16-byte load: {group | weight tile << 16 (-1: none), first row | narrow flag,
// group's first row in the sorted rows, group's row count}. list: the tile list (2 ints per
// entry); grp: per group (first row, row count).
__device__ __forceinline__ void write_dispatch(const int* list, const int2* grp, int n_all,
                                              int n_wide, int n_wtiles, int wt_cols, int b_lo,
                                              int b_hi, int E, int I, int Is, u32x4* table) {
  const int W = n_wide * n_wtiles, N = (n_all - n_wide) * n_wtiles;
  for (int b = b_lo + static_cast<int>(threadIdx.x); b < b_hi; b += blockDim.x) {
    const int item = dispatch_item(b, W, N);
    u32x4 ent = {0xffffffffu, 0u, 0u, 0u};
    if (item >= 0) {
      const int ti = item / n_wtiles, wt = item - ti * n_wtiles;
      const int g = list[2 * ti];
      // weight tiles past a narrower shared expert (gate_up: wt_cols = kWM/2 channels) idle
      if (wt_cols == 0 || wt * wt_cols < (g == E ? Is : I)) {
        const int2 gr = grp[g];
        ent = u32x4{static_cast<uint32_t>(g | (wt << 16)), static_cast<uint32_t>(list[2 * ti + 1]),
                    static_cast<uint32_t>(gr.x), static_cast<uint32_t>(gr.y)};
      }
    }
    table[b] = ent;
  }
}

// Tile lists up to this many entries are also assembled in LDS, where the dispatch tables
// read them back; longer ones are read back from memory. With the list in LDS, up to
// kBuildBlocks workgroups write the dispatch tables: each assembles the (short) list itself and
// writes its share of the entries, so the table loop (two 64-bit divisions per entry) does not
// hold one CU for the whole launch. Workgroup 0 alone writes the list, its counts and the queues.
constexpr int kLdsListEntries = 4096;
constexpr int kBuildBlocks = 32;
constexpr int kBuildEntriesPerBlock = 256;

// The tile list and dispatch tables, by workgroup bidx of nblocks (1024 threads each; see
// kBuildBlocks). offsets == nullptr: the groups' first rows are the exclusive scan of counts
// (E <= 1024), computed here.
__device__ __forceinline__ void build_tiles_body(const int32_t* __restrict__ counts,
                                                 const int32_t* __restrict__ offsets, int E,
                                                 int shared, int T, int sh_row0, int max_tiles,
                                                 int wide, int narrow, int tiny, int I, int Is,
                                                 int H, int grid_gu, int grid_dn,
                                                 int32_t* __restrict__ tiles, int bidx,
                                                 int nblocks) {
  __shared__ int wsum[16];
  __shared__ int s_list[2 * kLdsListEntries];
  __shared__ int2 s_grp[1025];
  __shared__ int s_first[1024];
  const int G = E + shared;
  const int tid = threadIdx.x;
  const bool in_lds = max_tiles <= kLdsListEntries;
  if (offsets == nullptr) {
    int ex;
    block_scan_1024(tid < E ? counts[tid] : 0, ex, wsum);
    if (tid < E) s_first[tid] = ex;
    __syncthreads();
  }
  const int per = (G + 1023) / 1024;
  const int lo = min(G, tid * per), hi = min(G, lo + per);
  int lw = 0, ln = 0, nw, nn, nt;
  for (int g = lo; g < hi; ++g) {
    const int n = g < E ? counts[g] : T;
    s_grp[g] = int2{g < E ? (offsets ? offsets[g] : s_first[g]) : sh_row0, n};
    group_tiles(n, wide, narrow, tiny, nw, nn, nt);
    lw += nw;
    ln += nn + nt;
  }
  int pw, pn;
  const int tw = block_scan_1024(lw, pw, wsum);
  const int tn = block_scan_1024(ln, pn, wsum);
  pn += tw;
  const bool lead = bidx == 0;
  auto put = [&](int pos, int g, int e) {
    if (pos >= max_tiles) return;
    if (lead) {
      tiles[2 * pos] = g;
      tiles[2 * pos + 1] = e;
    }
    if (in_lds) {
      s_list[2 * pos] = g;
      s_list[2 * pos + 1] = e;
    }
  };
  for (int g = lo; g < hi; ++g) {
    group_tiles(s_grp[g].y, wide, narrow, tiny, nw, nn, nt);
    for (int i = 0; i < nw; ++i) put(pw++, g, i * wide);
    for (int i = 0; i < nn; ++i) put(pn++, g, (nw * wide + i * narrow) | kNarrowFlag);
    if (nt) put(pn++, g, (nw * wide) | kTinyFlag);
  }
  const int n_all = min(tw + tn, max_tiles), n_wide = min(tw, max_tiles);
  if (lead && tid == 0) {
    tiles[2 * max_tiles] = n_all;
    tiles[2 * max_tiles + 1] = n_wide;
  }
  if (grid_gu + grid_dn == 0) return;
  if (lead && tid < 8) {
    // gate_up work queue of XCD x: its slots of the dispatch table (slot j = entry j * 8 + x)
    // that dispatch_item fills, and a counter from zero
    const int x = tid, n_wt = I > Is ? I / (kWM / 2) : Is / (kWM / 2);
    const int W = n_wide * n_wt, N = (n_all - n_wide) * n_wt;
    const int cw = (W + 7) >> 3, cn = (N + 7) >> 3;
    const int nw = min(W, min(W, x * cw) + cw) - min(W, x * cw);
    const int nn = min(N, min(N, x * cn) + cn) - min(N, x * cn);
    int32_t* q = queue_base(tiles, max_tiles, grid_gu, grid_dn);
    q[x * 64] = 0;
    q[8 * 64 + x] = nw + nn;
  }
  __syncthreads();                           // the list is complete (and visible to the block)
  const int* list = in_lds ? s_list : tiles;
  u32x4* tab = reinterpret_cast<u32x4*>(tiles + table_base(max_tiles));
  // this workgroup's share of the entries, gate_up's table then down's
  const int total = grid_gu + grid_dn, share = (total + nblocks - 1) / nblocks;
  const int b_lo = min(total, bidx * share), b_hi = min(total, b_lo + share);
  write_dispatch(list, s_grp, n_all, n_wide, I > Is ? I / (kWM / 2) : Is / (kWM / 2), kWM / 2,
                 min(b_lo, grid_gu), min(b_hi, grid_gu), E, I, Is, tab);
  write_dispatch(list, s_grp, n_all, n_wide, H / kWM, 0, max(b_lo - grid_gu, 0),
                 max(b_hi - grid_gu, 0), E, I, Is, tab + grid_gu);
}

__global__ __launch_bounds__(1024) void build_tiles_kernel(const int32_t* __restrict__ counts,
                                                           const int32_t* __restrict__ offsets,
                                                           int E, int shared, int T, int sh_row0,
                                                           int max_tiles, int wide, int narrow,
                                                           int tiny, int I, int Is, int H, int grid_gu,
                                                           int grid_dn, int32_t* __restrict__ tiles) {
  build_tiles_body(counts, offsets, E, shared, T, sh_row0, max_tiles, wide, narrow, tiny, I, Is,
                   H, grid_gu, grid_dn, tiles, blockIdx.x, gridDim.x);
}

// Last pass of the permutation of router_route_kernel's selection, with the tile list built in
// the same launch. Routing entries come in chunks c = s * nb + b (slot s, 64-token block b),
// which in this order follow the reference's (slot, token) order; hist/base hold per expert and
// chunk the count and the exclusive prefix (base, from perm_expert_scan) and lrank each entry's
// rank among its chunk's entries of the same expert. Workgroups below n_scatter place 16 chunks
// each (a wave per chunk, a lane per token), pos = first row of the expert + base + rank; the
// others build the tile list and dispatch tables from the expert totals.
__global__ __launch_bounds__(1024) void scatter_build_kernel(
    const int32_t* __restrict__ idx, int T, int k, int nb, const int32_t* __restrict__ base,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ lrank,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm_tok, int32_t* __restrict__ perm_slot,
    int32_t* __restrict__ inv, int n_scatter, int E, int shared, int sh_row0, int max_tiles,
    int wide, int narrow, int tiny, int I, int Is, int H, int grid_gu, int grid_dn,
    int32_t* __restrict__ tiles) {
  if (static_cast<int>(blockIdx.x) >= n_scatter) {
    build_tiles_body(counts, nullptr, E, shared, T, sh_row0, max_tiles, wide, narrow, tiny, I, Is,
                     H, grid_gu, grid_dn, tiles, blockIdx.x - n_scatter, gridDim.x - n_scatter);
    return;
  }
  __shared__ int wsum[16];
  __shared__ int s_off[1024];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  int ex;
  const int total = block_scan_1024(tid < E ? counts[tid] : 0, ex, wsum);
  if (tid < E) s_off[tid] = ex;
  if (blockIdx.x == 0) {
    if (tid < E) offsets[tid] = ex;
    if (tid == 0) offsets[E] = total;
  }
  __syncthreads();
  const int nchunks = k * nb, c = blockIdx.x * 16 + wave;
  if (c >= nchunks) return;
  const int s = c / nb, t = (c - s * nb) * 64 + lane;
  if (t >= T) return;
  const int64_t ts = static_cast<int64_t>(t) * k + s;
  const int e = idx[ts];                     // the router's own selection: always in [0, E)
  const int pos = s_off[e] + base[static_cast<int64_t>(e) * nchunks + c] +
                  lrank[static_cast<int64_t>(s) * T + t];
  perm_tok[pos] = t;
  perm_slot[pos] = s;
  inv[ts] = pos;
}

// The same for the chunks of launch_permute's count pass (perm_count): chunk c holds entries
// v = c * kPermChunk + r * 64 + lane (v = s * T + t, the reference's (slot, token) order) with
// their ranks in lrank. Scatter workgroup c places chunk c, wave r its round r (with
// 16 chunks per workgroup, as above, a prefill batch's few hundred chunks ran on a dozen CUs
// and the launch took longer than the scatter and tile build it replaced); ids outside [0, E)
// get inv = -1.
template <int IB>
__global__ __launch_bounds__(1024) void perm_scatter_build_kernel(
    const void* idx, int T, int k, int V, int nblk, const int32_t* __restrict__ base,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ lrank,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm_tok, int32_t* __restrict__ perm_slot,
    int32_t* __restrict__ inv, int n_scatter, int E, int shared, int sh_row0, int max_tiles,
    int wide, int narrow, int tiny, int I, int Is, int H, int grid_gu, int grid_dn,
    int32_t* __restrict__ tiles) {
  // the tile-list workgroups first, so that their work overlaps the scatter's
  const int n_build = static_cast<int>(gridDim.x) - n_scatter;
  if (static_cast<int>(blockIdx.x) < n_build) {
    build_tiles_body(counts, nullptr, E, shared, T, sh_row0, max_tiles, wide, narrow, tiny, I, Is,
                     H, grid_gu, grid_dn, tiles, blockIdx.x, n_build);
    return;
  }
  __shared__ int wsum[16];
  __shared__ int s_off[1024];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int c = static_cast<int>(blockIdx.x) - n_build;
  int ex;
  const int total = block_scan_1024(tid < E ? counts[tid] : 0, ex, wsum);
  if (tid < E) s_off[tid] = ex;
  if (c == 0) {
    if (tid < E) offsets[tid] = ex;
    if (tid == 0) offsets[E] = total;
  }
  __syncthreads();
  if (wave >= kPermChunk / kWave) return;
  const int v = c * kPermChunk + wave * kWave + lane;
  if (v >= V) return;
  const int s = v / T, t = v - s * T;
  const int64_t ts = static_cast<int64_t>(t) * k + s;
  const int e = load_expert<IB>(idx, ts);
  if (e < 0 || e >= E) {
    inv[ts] = -1;
    return;
  }
  const int pos = s_off[e] + base[static_cast<int64_t>(e) * nblk + c] + lrank[v];
  perm_tok[pos] = t;
  perm_slot[pos] = s;
  inv[ts] = pos;
}

// ---- one token tile --------------------------------------------------------------------------
// MODE kDown: out[row, h] = act[row] . Wd_g[h];  kGateUp: act[row, c] = silu(gate) * up;
// kRouter: logits[t, e] = x[t] . Wg[e] (gw.gate_up holds the router weight, gw.E its rows).
enum TileMode { kDown = 0, kGateUp = 1, kRouter = 2 };


// Rows r0 .. r0 + S::kWT - 1 (clipped to n) of group g (a routed expert, or the shared
// expert when g == gw.E), output columns of weight tile wt. row0: the group's first row in
// src (down) / dst.
// PERSIST: called from the persistent kernel, which passes its work queue. The tile then claims
// the next entry of the home queue after k-tile nk - 2's barrier, loads it at the start of the
// epilogue, and leaves it (or, when the claim found nothing, a synchronously fetched entry) in
// the ring's last 16 bytes, which no staged tile reaches.
// STAGE (router only): the tile's logits are also left in LDS, rounded to bf16, as rows of
// kStagedLogitStride entries per token (staged_logits), for a selection that follows in the
// same workgroup.
template <class S>
constexpr int kStagedLogitStride = S::kRows + 8;   // uint16 entries; + 8 against bank conflicts

// The router tile's accumulators (wave (wm, wn) of shape S) rounded to bf16 into LDS as rows of
// kStagedLogitStride entries per token, then the rows of its ne = min(S::kRows, E - c0) experts
// stored to dst (local token tl of the n - r0 left at row row0 + r0 + tl, dst_ld per row) with
// 16-byte lanes. Called by every thread of the workgroup once no wave reads lds any more.
template <class S>
__device__ __forceinline__ void stage_logits(const f32x16 (&acc)[S::kMT][S::kNT], int E, int n,
                                             int r0, int row0, int c0, uint16_t* __restrict__ dst,
                                             int dst_ld, u32x4* __restrict__ lds) {
  constexpr int kStride = kStagedLogitStride<S>, kMT = S::kMT, kNT = S::kNT, kRW = S::kRW;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w % S::kWavesM, wn = w / S::kWavesM;
  const int col = lane & 31, rq = 4 * (lane >> 5);
  ring_barrier();                                           // every wave is done with the ring
  uint16_t* sl = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int tl = wn * (kNT * 32) + 32 * t + col;          // token within the tile
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const int e = wm * kRW + 32 * i + 8 * v4 + rq;     // expert within the tile
        *reinterpret_cast<u32x2*>(sl + tl * kStride + e) =
            u32x2{pack_bf2(acc[i][t][4 * v4], acc[i][t][4 * v4 + 1]),
                  pack_bf2(acc[i][t][4 * v4 + 2], acc[i][t][4 * v4 + 3])};
      }
  }
  ring_barrier();
  const int ntok = min(S::kWT, n - r0), ne = min(S::kRows, E - c0);
  if ((ne & 7) == 0 && (dst_ld & 7) == 0 && (c0 & 7) == 0) {
    const int cpr = ne / 8;                                 // 16-byte chunks per row
    for (int i = threadIdx.x; i < ntok * cpr; i += kThreads) {
      const int tl = i / cpr, c = i - tl * cpr;
      *reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(row0 + r0 + tl) * dst_ld + c0 + 8 * c) =
          *reinterpret_cast<const u32x4*>(sl + tl * kStride + 8 * c);
    }
  } else {
    for (int i = threadIdx.x; i < ntok * ne; i += kThreads) {
      const int tl = i / ne, e = i - tl * ne;
      dst[static_cast<int64_t>(row0 + r0 + tl) * dst_ld + c0 + e] = sl[tl * kStride + e];
    }
  }
}

// Partial sums of a router tile over a k range, in fp32: accumulator element 4 q + v of tile
// (i, t) of wave w, lane l lands at float (((((i * kNT + t) * 4 + q) * kWaves + w) * 64 + l) * 4
// + v, so every store and load instruction moves 1 KB of consecutive bytes.
template <class S>
constexpr int kPartialFloats = S::kMT * S::kNT * 16 * kThreads;
template <class S>
__device__ __forceinline__ void store_partial(const f32x16 (&acc)[S::kMT][S::kNT],
                                              float* __restrict__ part) {
  f32x4* p = reinterpret_cast<f32x4*>(part) + threadIdx.x;
#pragma unroll
  for (int i = 0; i < S::kMT; ++i)
#pragma unroll
    for (int t = 0; t < S::kNT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        p[((i * S::kNT + t) * 4 + q) * kThreads] =
            f32x4{acc[i][t][4 * q], acc[i][t][4 * q + 1], acc[i][t][4 * q + 2], acc[i][t][4 * q + 3]};
}
// PARTIAL (router only): only k-tiles kt0 .. kt0 + nkt - 1 of the product, whose fp32 sums go
// to part (store_partial) instead of logits.
template <int MODE, class S, int kLdsCap = kLdsU4, bool PERSIST = false, bool STAGE = false,
          bool PARTIAL = false>
__device__ __forceinline__ void tile_product(const GroupWeights& gw, const uint16_t* __restrict__ src,
                                             int src_ld, const int32_t* __restrict__ perm_tok,
                                             int g, int r0, int n, int row0, int wt,
                                             uint16_t* __restrict__ dst, int dst_ld,
                                             u32x4* __restrict__ lds, WorkQueue* wq = nullptr,
                                             int kt0 = 0, int nkt = 0,
                                             float* __restrict__ part = nullptr) {
  constexpr bool GATEUP = MODE == kGateUp, ROUTER = MODE == kRouter;
  constexpr int kMT = S::kMT, kNT = S::kNT, kRW = S::kRW, kWavesM = S::kWavesM;
  constexpr int kBK = S::kBK, kStages = S::kStages, kChunks = S::kChunks;
  constexpr int kRowsPerLoad = S::kRowsPerLoad, kALoads = S::kALoads, kBLoads = S::kBLoads;
  constexpr int kLoads = S::kLoads, kKSteps = S::kKSteps;
  constexpr int kSwzShift = S::kSwzShift;
  constexpr int kRows = S::kRows;                  // weight rows of the tile
  static_assert(ROUTER || kRows == kWM, "expert GEMMs take kWM weight rows per tile");
  static_assert(!GATEUP || kMT % 2 == 0, "gate_up pairs a wave's gate tiles with its up tiles");
  static_assert(!PARTIAL || (ROUTER && !STAGE), "partial sums are router tiles");
  const bool shared = !ROUTER && g == gw.E;
  const int Ig = shared ? gw.Is : gw.I;
  const int H = gw.H;
  const int K = (GATEUP || ROUTER) ? H : Ig;
  const int c0 = wt * (GATEUP ? kRows / 2 : kRows);  // first channel / output column

  // In the persistent kernel's item loop the thread index goes through an empty asm, so the
  // per-lane address arithmetic below is redone per item instead of being hoisted out of the
  // loop and held in registers across the main loop (which spilled).
  int tid = threadIdx.x;
  if constexpr (PERSIST) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  // Wave index as a scalar: LDS destinations of the copies (M0) are then computed on the SALU.
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w % kWavesM, wn = w / kWavesM;

  // Direct global->LDS copies: wave copy i writes one contiguous 1 KB LDS block of
  // kRowsPerLoad rows; lane l fills slot l of it, i.e. row R0 + l/kChunks at swizzled position
  // l%kChunks, so it fetches the chunk that the swizzle places there. The copies go through
  // buffer resources (buffer_load ... lds): a wave-uniform descriptor per copy, a fixed 32-bit
  // byte offset per lane, and the k-tile's step in the scalar offset. With global_load_lds the
  // compiler counted the copies as LDS operations as well and then waited for every
  // outstanding LDS read (lgkmcnt(0)) before each k-step's first MFMA; buffer copies leave the
  // LDS reads in order for it, so each MFMA waits only for its own fragments. Byte offsets stay
  // below 2^31 (tiled_offsets_fit on the host).
  static_assert(32 % kRowsPerLoad == 0, "a copy's rows lie in one 32-row block");
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
  __amdgpu_buffer_rsrc_t ars[kALoads];
  uint32_t aoff[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int row0c = (w * kALoads + i) * kRowsPerLoad;          // the copy's first row (uniform)
    const int row = row0c + lrow;                                // local weight row
    const int j = lpos ^ ((row >> kSwzShift) & (kChunks - 1));
    int grow;
    const uint16_t* base = wbase;
    if (GATEUP) {
      // 32-row blocks alternate the gate and the up rows of 32 channels: block b holds channels
      // c0 + 32 (b / 2) .. +32, gate rows for even b, up rows for odd b, so MFMA tiles 2p and
      // 2p + 1 of a wave pair up in every tile shape
      base = ((row0c >> 5) & 1) ? wup : wbase;
      grow = c0 + 32 * (row >> 6) + (row & 31);
    } else if (ROUTER) {
      grow = min(c0 + row, gw.E - 1);      // rows past E repeat a valid row; not stored
    } else {
      grow = c0 + row;
    }
    ars[i] = raw_rsrc(base);
    aoff[i] = static_cast<uint32_t>((static_cast<int64_t>(grow) * K + 8 * j) * 2);
    if constexpr (PARTIAL) aoff[i] += static_cast<uint32_t>(kt0 * kBK * 2);
  }
  // Weight bytes between k-tile kt and kt + 1 of a copy: kBK elements along the checkpoint
  // rows, or one whole k-tile block in the tiled layout (pack_tiled_kernel), where the kWM x
  // kBK k-tile is a contiguous 32 KB block in LDS order, so wave copy i reads the 1 KB at slot
  // (w * kALoads + i) * 64 of it, lane l the 16 bytes of slot l.
  int astep = kBK * 2;
  if constexpr (!ROUTER) {
    const void* tl = GATEUP ? (shared ? gw.sh_gate_up_tiled : gw.gate_up_tiled)
                            : (shared ? gw.sh_down_tiled : gw.down_tiled);
    if (tl != nullptr) {
      const int64_t group = shared ? 0 : static_cast<int64_t>(g) * (GATEUP ? 2 : 1) * Ig * H;
      const uint16_t* wtl = static_cast<const uint16_t*>(tl) + group + static_cast<int64_t>(wt) * kWM * K;
      astep = kWM * kBK * 2;
#pragma unroll
      for (int i = 0; i < kALoads; ++i) {
        ars[i] = raw_rsrc(wtl);
        aoff[i] = static_cast<uint32_t>(((w * kALoads + i) * (kRowsPerLoad * kChunks) + lane) * 16);
      }
    }
  }
  const __amdgpu_buffer_rsrc_t brs = raw_rsrc(src);
  uint32_t boff[kBLoads];
#pragma unroll
  for (int i = 0; i < kBLoads; ++i) {
    const int lt = (w * kBLoads + i) * kRowsPerLoad + lrow;     // local token
    const int row = kRows + lt;
    const int j = lpos ^ ((row >> kSwzShift) & (kChunks - 1));
    const int p = min(r0 + lt, n - 1);   // rows past the group repeat a valid row; not stored
    const int srow = ROUTER ? p : (GATEUP ? (shared ? p : perm_tok[row0 + p]) : row0 + p);
    boff[i] = static_cast<uint32_t>((static_cast<int64_t>(srow) * src_ld + 8 * j) * 2);
    if constexpr (PARTIAL) boff[i] += static_cast<uint32_t>(kt0 * kBK * 2);
  }

  f32x16 acc[kMT][kNT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  typedef __attribute__((address_space(3))) void* lds_ptr;
  // Narrow and tiny tiles serve experts whose weights no other token tile reads: their weight
  // copies are non-temporal (cache policy nt), so the stream does not displace the token rows
  // and wide-tile weights that are reused (E=512 T=4096 layer 755 -> 727 us, Qwen3-30B-A3B
  // T=8192 Zipf 763 -> 741 us; the same for every tile was slower, 766 -> 799 us).
  constexpr int kWeightPolicy = (!ROUTER && S::kWT < kWM) ? 2 : 0;
  // the copies of k-tile kt into ring stage `stage`
  auto issue_a = [&](int stage, int kt) {
    u32x4* buf = lds + S::a_off(stage);
#pragma unroll
    for (int i = 0; i < kALoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ars[i], (lds_ptr)(buf + (w * kALoads + i) * kRowsPerLoad * kChunks), 16, aoff[i],
          kt * astep, 0, kWeightPolicy);
  };
  auto issue_b = [&](int stage, int kt) {
    u32x4* buf = lds + S::b_off(stage);
#pragma unroll
    for (int i = 0; i < kBLoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          brs, (lds_ptr)(buf + ((w * kBLoads + i) * kRowsPerLoad) * kChunks), 16, boff[i],
          kt * (kBK * 2), 0, 0);
  };
  auto issue = [&](int stage, int kt) {
    issue_a(stage, kt);
    issue_b(stage, kt);
  };

  // Ring protocol (the asymmetric ring issues A0 B0 A1 B1 A2 up front, then refills B kt+2
  // and A kt+3 after k-tile kt, so at the end of k-tile kt only A kt+2 is younger than the
  // copies of k-tile kt+1). Otherwise all kStages buffers are filled up front. In k-tile kt, once this wave
  // has read the last k-step's fragments of stage kt, it waits for its copies of stage kt+1,
  // meets the other waves at the barrier (after which nobody reads stage kt any more), reads
  // stage kt+1's first fragments and refills stage kt's buffer with k-tile kt+kStages, all
  // interleaved with the last k-step's MFMAs, so neither the copy issue nor the LDS read
  // latency of the next k-tile stands between two MFMAs.
  const int nk = PARTIAL ? nkt : K / kBK;
  // Wide expert tiles (MFMA-bound) put only stage 0 out before the first wait. A wave reaches
  // its wait once it has issued every copy before it, and the CU's copy path takes the waves'
  // copies in turn: with the whole ring issued up front, the second wave of each SIMD saw its
  // stage 0 land only after the path had drained the entire fill (160 KB; 1.9 instead of
  // 1.2 us). Their other stages follow in k-tile 0 (fill_stage), in the same order as up
  // front, so every later wait counts the same younger copies. Narrow and tiny tiles are
  // bound by HBM and keep the whole fill up front: stages issued later cost them more than the
  // earlier start gains (E=512 T=4096 down 240 -> 243 us). There a barrier after stage 0 puts
  // every wave's stage 0 on the copy path before any wave's later stages.
  constexpr bool kLazyFill = !ROUTER && S::kWT == kWM;
  // Stage st's copies of the fill, in the order of the asymmetric ring (A0 B0 A1 B1 A2) or the
  // symmetric one (A0 B0 A1 B1 A2 B2 ...). CHECK: nk may be at most st.
  auto fill_stage = [&]<bool CHECK>(int st) {
    if (!CHECK || st < nk) issue_a(st, st);
    if (st < S::kBStages && (!CHECK || st < nk)) issue_b(st, st);
  };
  if constexpr (kLazyFill) {
    issue(0, 0);
  } else {
#pragma unroll
    for (int st = 0; st < kStages; ++st) {
      fill_stage.template operator()<true>(st);
      if (st == 0) ring_barrier();
    }
  }
  const int mr = lane & 31, mk = lane >> 5;   // MFMA operand: row l%32, k-chunk half l/32
  auto read_frags = [&](int kt, int ks, u32x4 (&fa)[kMT], u32x4 (&fb)[kNT]) {
    const int j = 2 * ks + mk;
    const u32x4* ca = lds + S::a_off(kt % kStages);
    const u32x4* cb = lds + S::b_off(kt % S::kBStages);
    // token fragments first: every MFMA of the k-step needs one, so the next k-step's first
    // MFMA then waits only for the oldest reads, not for the whole batch
#pragma unroll
    for (int t = 0; t < kNT; ++t) fb[t] = cb[S::swz(wn * (kNT * 32) + 32 * t + mr, j)];
#pragma unroll
    for (int i = 0; i < kMT; ++i) fa[i] = ca[S::swz(wm * kRW + 32 * i + mr, j)];
  };
  auto mfma_all = [&](const u32x4 (&fa)[kMT], const u32x4 (&fb)[kNT]) {
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int t = 0; t < kNT; ++t)
        acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(fa[i]), as_bf16x8(fb[t]),
                                                            acc[i][t], 0, 0, 0);
  };
  constexpr int kReads = kMT + kNT, kMfmas = kMT * kNT;
  constexpr int kPaired = kReads < kMfmas ? kReads : kMfmas;
  // fragment reads one-for-one with the first MFMAs (leftover reads after them)
  auto sched_reads = [&]() {
#pragma unroll
    for (int r = 0; r < kPaired; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (kReads > kPaired) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPaired, 0);
  };
  u32x4 fa[2][kMT], fb[2][kNT];
  // One k-tile. NEXT: a k-tile follows (wait, barrier, read its first fragments); REFILL: the
  // freed buffers take k-tile kt + kStages (2: both operands; 1: the asymmetric ring's token
  // operand only, whose ring runs one k-tile shorter). FILL (k-tile 0 when nk > kStages): the
  // ring's stages 1 .. kStages - 1 go out behind the MFMAs of the first k-steps, one stage per
  // k-step. Specialised at compile time so that the loop body has no branches around the MFMAs.
  static_assert(kStages <= kKSteps, "the fill issues one stage per k-step of k-tile 0");
  int claim = -1;      // PERSIST: home-queue slot claimed for the next item (-1: none)
  auto ktile = [&]<bool NEXT, int REFILL, bool CLAIM = false, bool FILL = false>(int kt) {
#pragma unroll
    for (int ks = 0; ks + 1 < kKSteps; ++ks) {
      read_frags(kt, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      mfma_all(fa[ks & 1], fb[ks & 1]);
      constexpr int kRest = kMfmas - kPaired;
      if (FILL && ks + 1 < kStages) {
        fill_stage.template operator()<false>(ks + 1);
        sched_reads();
        constexpr int kPer = (kLoads + (kRest > 0 ? kRest : 1) - 1) / (kRest > 0 ? kRest : 1);
#pragma unroll
        for (int r = 0; r < kRest; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, kPer, 0);
        }
        if constexpr (kRest == 0) __builtin_amdgcn_sched_group_barrier(0x020, kLoads, 0);
      } else {
        sched_reads();
        if constexpr (kRest > 0) __builtin_amdgcn_sched_group_barrier(0x008, kRest, 0);
      }
    }
    constexpr int kl = (kKSteps - 1) & 1;
    if constexpr (NEXT) {
      // all earlier MFMAs stay above the barrier: they cover the last fragment reads' latency
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (S::kAsym) {
        // k-tile kt+1 must have landed; only the weight copies of k-tile kt+2 may be younger
        if (kt + 2 < nk) wait_vmcnt<kALoads>();
        else wait_vmcnt<0>();
      } else {
        wait_ring<kStages - 2, kLoads>(nk - 2 - kt);
      }
      ring_barrier();
      read_frags(kt + 1, 0, fa[0], fb[0]);
      if constexpr (S::kAsym) {
        if constexpr (REFILL >= 1) issue_b(kt % S::kBStages, kt + S::kBStages);
        if constexpr (REFILL >= 2) issue_a(kt % kStages, kt + kStages);
      } else {
        if constexpr (REFILL >= 2) issue(kt % kStages, kt + kStages);
      }
      if constexpr (CLAIM) {
        // Every copy has landed (the wait above), so no ring wait counts the atomic. Through an
        // address the compiler cannot prove uniform it stays a plain atomic whose result is
        // waited for at its first use in the epilogue; the wave-level form it would otherwise
        // take reads the result back right here.
        if (threadIdx.x == 0 && wq->tried == 0) {
          int* cnt = wq->q + wq->home * 64;
          asm volatile("" : "+v"(cnt));
          claim = __hip_atomic_fetch_add((__attribute__((address_space(1))) int*)cnt, 1,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    mfma_all(fa[kl], fb[kl]);
    if constexpr (NEXT) {
      // next k-tile's first reads with the first MFMAs, then the copies spread over the rest
      sched_reads();
      constexpr int kRest = kMfmas - kPaired;
      if constexpr (REFILL > 0 && kRest > 0) {
        constexpr int kPer = (kLoads + kRest - 1) / (kRest > 0 ? kRest : 1);
#pragma unroll
        for (int r = 0; r < kRest; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, kPer, 0);
        }
      }
    }
  };
  if constexpr (kLazyFill) {
    wait_vmcnt<0>();                   // stage 0, the only copies out
  } else if constexpr (S::kAsym) {
    // k-tile 0 must have landed; younger: k-tile 1 (both operands) and k-tile 2's weights
    if (nk > 2) wait_vmcnt<kLoads + kALoads>();
    else if (nk > 1) wait_vmcnt<kLoads>();
    else wait_vmcnt<0>();
  } else {
    wait_ring<kStages - 1, kLoads>(nk - 1);
  }
  ring_barrier();
  read_frags(0, 0, fa[0], fb[0]);
  int kt = 0;
  if constexpr (kLazyFill) {
    if (nk > kStages) {
      ktile.template operator()<true, 2, false, true>(kt++);
    } else {
#pragma unroll
      for (int st = 1; st < kStages; ++st) fill_stage.template operator()<true>(st);
    }
  }
  for (; kt + kStages < nk; ++kt) ktile.template operator()<true, 2>(kt);
  if constexpr (S::kAsym)
    for (; kt + S::kBStages < nk; ++kt) ktile.template operator()<true, 1>(kt);
  if constexpr (PERSIST) {
    // k-tile nk - 2 claims the next item; outside the loop the claim's register is not carried
    // around a loop edge, where the compiler copied it (and waited for the atomic) at once
    for (; kt + 2 < nk; ++kt) ktile.template operator()<true, 0>(kt);
    if (kt + 1 < nk) ktile.template operator()<true, 0, true>(kt++);
  } else {
    for (; kt + 1 < nk; ++kt) ktile.template operator()<true, 0>(kt);
  }
  ktile.template operator()<false, 0>(kt);

  // Epilogue.
  const int col = lane & 31, rq = 4 * (lane >> 5);
  if constexpr (!ROUTER) {
    // Stage the tile in LDS as row-major [token][column] bf16, then store whole row segments
    // (kCols * 2 contiguous bytes per token) with 16-byte lanes. Storing straight from the
    // accumulators would write 16-byte pieces of 32 token rows per instruction.
    constexpr int kCols = GATEUP ? kWM / 2 : kWM;            // output columns per tile
    static_assert(S::kWT * (kCols / 8) <= kLdsCap, "staged tile exceeds the LDS ring");
    ring_barrier();                                           // every wave is done with the ring
    u32x4 next = {0xffffffffu, 0u, 0u, 0u};
    if constexpr (PERSIST) {
      static_assert(S::kWT * (kCols / 8) < kLdsCap, "the staged tile covers the next-item slot");
      // the claimed entry's load goes out here and is used after the staging writes; the empty
      // asm keeps the claim's first use (with the wait for the atomic) from moving up into the
      // last k-tile
      if (threadIdx.x == 0) {
        asm volatile("" : "+v"(claim));
        if (claim >= 0 && claim < wq->own_len) next = wq->table[claim * 8 + wq->home];
      }
    }
    char* st = reinterpret_cast<char*>(lds);
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int r = wn * (kNT * 32) + 32 * t + col;           // token within the tile
#pragma unroll
      for (int i = 0; i < (GATEUP ? kMT / 2 : kMT); ++i)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          float a[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            a[v] = GATEUP ? silu(acc[2 * i][t][4 * v4 + v]) * acc[2 * i + 1][t][4 * v4 + v]
                          : acc[i][t][4 * v4 + v];
          const int c = (GATEUP ? wm * (kRW / 2) : wm * kRW) + 32 * i + 8 * v4 + rq;
          *reinterpret_cast<u32x2*>(st + staged_slot<kCols>(r, c / 8) * 16 + (c % 8) * 2) =
              u32x2{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
        }
    }
    if constexpr (PERSIST) {
      if (threadIdx.x == 0) {
        if (static_cast<int>(next[0]) < 0) {
          // no claim, a claim past the home queue's end (the queue is then empty), or an idle
          // entry: fetch synchronously
          if (claim >= wq->own_len) wq->tried = wq->tried > 1 ? wq->tried : 1;
          next = queue_fetch(*wq);
        }
        lds[kLdsCap - 1] = next;
      }
    }
    ring_barrier();
    store_staged<kCols, S::kWT, !GATEUP>(lds, dst, dst_ld, row0, r0, n, c0);   // down: read once
  } else if constexpr (PARTIAL) {
    store_partial<S>(acc, part);
  } else if constexpr (STAGE) {
    // logits through LDS: staged rows, then whole rows stored with 16-byte lanes
    static_assert(S::kWT * kStagedLogitStride<S> * 2 <= kLdsCap * 16, "staged logits exceed the ring");
    stage_logits<S>(acc, gw.E, n, r0, row0, c0, dst, dst_ld, lds);
  } else {
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int p = r0 + wn * (kNT * 32) + 32 * t + col;
      if (p >= n) continue;
      uint16_t* orow = dst + static_cast<int64_t>(row0 + p) * dst_ld;
      const int E = gw.E;
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const int e = c0 + wm * kRW + 32 * i + 8 * v4 + rq;
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
    }
  }
}

// ---- the kernels -----------------------------------------------------------------------------
// Router logits: one workgroup per (token tile of S::kWT, weight tile of S::kRows experts), no
// tile list.
template <class S>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 4)))
void router_tiled_kernel(GroupWeights gw, const uint16_t* __restrict__ x, int T, int n_wtiles,
                         uint16_t* __restrict__ logits) {
  __shared__ u32x4 lds[S::kRingU4];
  const int logical = xcd_item(blockIdx.x, (T + S::kWT - 1) / S::kWT * n_wtiles);
  if (logical < 0) return;
  const int ti = logical / n_wtiles, wt = logical - ti * n_wtiles;
  tile_product<kRouter, S, S::kRingU4>(gw, x, gw.H, nullptr, 0, ti * S::kWT, T, 0,
                                                     wt, logits, gw.E, lds);
}

constexpr int kRouteMaxK = 16;
// LDS of the selection: the staged logits of a 64-token block, then the ids and per-wave counts.
constexpr int kRouteStagedBytes = RouterShape128::kWT * kStagedLogitStride<RouterShape128> * 2;
constexpr int kRouteLdsBytes =
    kRouteStagedBytes + (RouterShape128::kWT * kRouteMaxK + kWaves * RouterShape128::kRows) * 4;
static_assert(kRouteStagedBytes % 16 == 0 && kRouteLdsBytes % 16 == 0, "16-byte LDS units");

// Selection and the first permutation pass of 64-token block b (E <= 128) from its logits,
// staged in lds by stage_logits: each wave selects 8 tokens at once (route_select8, an 8-lane
// group per token, experts 8j + u on lane u of the group) and keeps their ids in LDS; then, for
// each slot s, a wave ranks the block's 64 entries of chunk c = s * nb + b among equal experts
// (ballot match, in token order) into lrank and writes the chunk's per-expert counts to
// hist[e * k * nb + c]. perm_expert_scan and scatter_build_kernel finish the sort. EPG: experts
// per lane, ceil(E / 8) rounded up to 8 or 16.
template <int EPG>
__device__ __forceinline__ void route_block(const uint16_t* __restrict__ x, int T, int E, int H,
                                            const float* __restrict__ bias,
                                            const uint16_t* __restrict__ w_sg, int k, int nbits,
                                            int nb, int b, int32_t* __restrict__ idx,
                                            uint16_t* __restrict__ topw, float* __restrict__ sgate,
                                            int32_t* __restrict__ hist,
                                            int32_t* __restrict__ lrank, u32x4* lds) {
  using S = RouterShape128;
  constexpr int kStride = kStagedLogitStride<S>, kPerWave = S::kWT / kWaves;
  static_assert(kPerWave == kWave / 8, "a wave selects one token per 8-lane group");
  static_assert(8 * EPG <= S::kRows, "experts per lane exceed the tile");
  int32_t* s_idx = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(lds) + kRouteStagedBytes);
  int32_t* s_cnt = s_idx + S::kWT * kRouteMaxK;              // [kWaves][S::kRows]
  const int t0 = b * S::kWT, nt = min(S::kWT, T - t0);
  const uint16_t* sl = reinterpret_cast<const uint16_t*>(lds);
  const int lane = lane_id(), u = lane & 7;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (sgate != nullptr) {
    // the shared-expert gate of the wave's tokens, a whole wave per token
    for (int i = 0; i < kPerWave; ++i) {
      const int tl = w * kPerWave + i;                        // the same for the whole wave
      if (tl >= nt) break;
      shared_gate(x, w_sg, t0 + tl, H, sgate);
    }
  }
  const int tl = w * kPerWave + (lane >> 3);                  // this lane group's token
  const bool ok = tl < nt;
  const int tr = ok ? tl : 0;                                 // past the batch: token 0's row
  float z[EPG];
#pragma unroll
  for (int j = 0; j < EPG; ++j) {
    const int e = 8 * j + u, ec = min(e, E - 1);
    const float v = bf2f(sl[tr * kStride + ec]) + (bias ? bias[ec] : 0.f);
    z[j] = (!(v == v) || e >= E) ? -INFINITY : v;             // a NaN logit is never preferred
  }
  route_select8<EPG>(z, E, k, static_cast<int64_t>(t0 + tl) * k, ok, idx, topw, s_idx + tr * k,
                     bias == nullptr);
  __syncthreads();
  const int nchunks = k * nb;
  for (int s = w; s < k; s += kWaves) {
    const int c = s * nb + b;
    int32_t* cnt = s_cnt + w * S::kRows;
    for (int e = lane; e < E; e += kWave) cnt[e] = 0;
    const bool valid = lane < nt;
    const int e = valid ? s_idx[lane * k + s] : 0;            // in [0, E): the selection's own
    const uint64_t m = match_expert(e, __ballot(valid), nbits);
    const int rank = mask_rank(m);
    if (valid) {
      lrank[static_cast<int64_t>(s) * T + t0 + lane] = rank;
      if (rank == 0) cnt[e] = __popcll(m);                  // a wave's LDS accesses are in order
    }
    for (int e2 = lane; e2 < E; e2 += kWave)
      hist[static_cast<int64_t>(e2) * nchunks + c] = cnt[e2];
  }
}

// Router logits, selection and the first permutation pass in one workgroup per 64-token block
// b (E <= 128, so one tile holds every expert): the tile's logits stay in LDS (STAGE) for
// route_block. Saves the route and count launches and the logits' round trip.
template <int EPG>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 4)))
void router_route_kernel(GroupWeights gw, const uint16_t* __restrict__ x, int T,
                         const float* __restrict__ bias, const uint16_t* __restrict__ w_sg, int k,
                         int nbits, int nb, uint16_t* __restrict__ logits, int32_t* __restrict__ idx,
                         uint16_t* __restrict__ topw, float* __restrict__ sgate,
                         int32_t* __restrict__ hist, int32_t* __restrict__ lrank) {
  using S = RouterShape128;
  // The ring is the kernel's only LDS object: the ids and counts live in it, behind the staged
  // logits. With a second __shared__ array in the kernel the compiler made every LDS read of
  // the k-loop wait for all global->LDS copies in flight (s_waitcnt vmcnt(0)), which drained
  // the ring each k-tile (the tile took 30 instead of 19 us at Qwen3-30B-A3B T=8192).
  __shared__ u32x4 lds[S::kRingU4];
  static_assert(kRouteLdsBytes <= S::kRingU4 * 16, "ids and counts exceed the ring");
  const int b = xcd_item(blockIdx.x, nb);
  if (b < 0) return;
  tile_product<kRouter, S, S::kRingU4, false, true>(gw, x, gw.H, nullptr, 0, b * S::kWT, T, 0, 0,
                                                    logits, gw.E, lds);
  route_block<EPG>(x, T, gw.E, gw.H, bias, w_sg, k, nbits, nb, b, idx, topw, sgate, hist, lrank,
                   lds);
}

// The same work in two launches where the blocks alone would leave CUs idle (small and mid-size
// batches): the tile's per-workgroup time is set by the bytes it streams (the whole router
// weight, 512 KB at E = 128, H = 2048, plus its tokens' rows), whatever the batch, so the k
// range is split. router_partial_kernel: workgroup (b, p) forms block b's fp32 sums over
// k-tiles [p nkt, (p + 1) nkt) into part + (b * splits + p) * kPartialFloats.
// router_select_kernel: block b's workgroup adds its splits' sums in p order (a fixed order,
// so the logits do not depend on timing), rounds them to bf16 and runs route_block.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 4)))
void router_partial_kernel(GroupWeights gw, const uint16_t* __restrict__ x, int T, int nb,
                           int splits, float* __restrict__ part) {
  using S = RouterShape128;
  __shared__ u32x4 lds[S::kRingU4];
  const int item = xcd_item(blockIdx.x, nb * splits);
  if (item < 0) return;
  const int b = item / splits, p = item - b * splits;
  const int nkt = gw.H / S::kBK / splits;
  tile_product<kRouter, S, S::kRingU4, false, false, true>(
      gw, x, gw.H, nullptr, 0, b * S::kWT, T, 0, 0, nullptr, 0, lds, nullptr, p * nkt, nkt,
      part + static_cast<int64_t>(item) * kPartialFloats<S>);
}

template <int EPG, int SPLITS>
__global__ __launch_bounds__(kThreads)
void router_select_kernel(GroupWeights gw, const uint16_t* __restrict__ x, int T,
                          const float* __restrict__ part, const float* __restrict__ bias,
                          const uint16_t* __restrict__ w_sg, int k, int nbits, int nb,
                          uint16_t* __restrict__ logits, int32_t* __restrict__ idx,
                          uint16_t* __restrict__ topw, float* __restrict__ sgate,
                          int32_t* __restrict__ hist, int32_t* __restrict__ lrank) {
  using S = RouterShape128;
  static_assert(S::kMT == 1 && S::kNT == 1, "one accumulator tile per wave");
  __shared__ u32x4 lds[kRouteLdsBytes / 16];
  const int b = xcd_item(blockIdx.x, nb);
  if (b < 0) return;
  // every split's four 16-byte pieces in flight at once, then the sums in split order
  const f32x4* pp = reinterpret_cast<const f32x4*>(part) +
                    static_cast<int64_t>(b) * SPLITS * (kPartialFloats<S> / 4) + threadIdx.x;
  f32x4 v[SPLITS][4];
#pragma unroll
  for (int p = 0; p < SPLITS; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) v[p][q] = pp[(p * 4 + q) * kThreads];
  f32x16 acc[1][1];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 a = v[0][q];
#pragma unroll
    for (int p = 1; p < SPLITS; ++p) a += v[p][q];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[0][0][4 * q + j] = a[j];
  }
  stage_logits<S>(acc, gw.E, T, b * S::kWT, 0, 0, logits, gw.E, lds);
  route_block<EPG>(x, T, gw.E, gw.H, bias, w_sg, k, nbits, nb, b, idx, topw, sgate, hist, lrank,
                   lds);
}

// explicit instantiations: with only the two launches in launch_router_route, the host pass left
// the second one's launch stub undefined in the library
template __global__ void router_route_kernel<8>(GroupWeights, const uint16_t*, int, const float*,
                                                const uint16_t*, int, int, int, uint16_t*,
                                                int32_t*, uint16_t*, float*, int32_t*, int32_t*);
template __global__ void router_route_kernel<16>(GroupWeights, const uint16_t*, int, const float*,
                                                const uint16_t*, int, int, int, uint16_t*,
                                                int32_t*, uint16_t*, float*, int32_t*, int32_t*);
#define LBMOE_SELECT_INST(EPG, SPLITS)                                                          \
  template __global__ void router_select_kernel<EPG, SPLITS>(                                  \
      GroupWeights, const uint16_t*, int, const float*, const float*, const uint16_t*, int, int, \
      int, uint16_t*, int32_t*, uint16_t*, float*, int32_t*, int32_t*);
LBMOE_SELECT_INST(8, 2)
LBMOE_SELECT_INST(8, 4)
LBMOE_SELECT_INST(16, 2)
LBMOE_SELECT_INST(16, 4)
#undef LBMOE_SELECT_INST

template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tiled_kernel(GroupWeights gw, const uint16_t* __restrict__ src, int src_ld,
                  const int32_t* __restrict__ perm_tok, const u32x4* __restrict__ table, int T,
                  uint16_t* __restrict__ dst, int dst_ld) {
  __shared__ u32x4 lds[kLdsU4];
  const TileItem it = decode_item(table[blockIdx.x]);
  if (it.g < 0) return;
  if (it.tiny)
    tile_product<MODE, Tiny>(gw, src, src_ld, perm_tok, it.g, it.r0, it.n, it.row0, it.wt, dst,
                             dst_ld, lds);
  else if (it.narrow)
    tile_product<MODE, Narrow>(gw, src, src_ld, perm_tok, it.g, it.r0, it.n, it.row0, it.wt,
                               dst, dst_ld, lds);
  else
    tile_product<MODE, Wide>(gw, src, src_ld, perm_tok, it.g, it.r0, it.n, it.row0, it.wt, dst,
                             dst_ld, lds);
}

// Persistent form of tiled_kernel: one workgroup per CU takes the dispatch-table entries from
// the per-XCD work queues until they run dry. The hardware hands a launch's workgroups to an
// XCD strictly in order, each to the next of its four shader engines in turn, so a CU that
// finishes a short (HBM-bound) item waits until the workgroups ahead of the next one have found
// CUs in their own shader engines; with wide items of ~53 us next to tiny ones of ~28 us, CUs of
// the gate_up launch sat idle for 14% of its span. Taken from a queue, an item starts on
// whichever CU of the XCD frees up first.
template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void tiled_persistent_kernel(GroupWeights gw, const uint16_t* __restrict__ src, int src_ld,
                             const int32_t* __restrict__ perm_tok, const u32x4* __restrict__ table,
                             int slots, int* __restrict__ q, uint16_t* __restrict__ dst,
                             int dst_ld) {
  __shared__ u32x4 lds[kLdsU4];
  const int home = blockIdx.x & 7;                 // workgroup b runs on XCD b % 8
  WorkQueue wq{table, slots, q, home, 0, 0};
  if (threadIdx.x == 0) {
    wq.own_len = min(q[8 * 64 + home], slots);
    lds[kLdsU4 - 1] = queue_fetch(wq);
  }
  for (;;) {
    ring_barrier();                    // the entry is in LDS, and the last tile's staging is read
    const TileItem it = decode_item(lds[kLdsU4 - 1]);
    ring_barrier();                    // every wave has the entry before the ring overwrites it
    if (it.g < 0) break;               // the same for the whole workgroup
    if (it.tiny)
      tile_product<MODE, Tiny, kLdsU4, true>(gw, src, src_ld, perm_tok, it.g, it.r0, it.n,
                                             it.row0, it.wt, dst, dst_ld, lds, &wq);
    else if (it.narrow)
      tile_product<MODE, Narrow, kLdsU4, true>(gw, src, src_ld, perm_tok, it.g, it.r0, it.n,
                                               it.row0, it.wt, dst, dst_ld, lds, &wq);
    else
      tile_product<MODE, Wide, kLdsU4, true>(gw, src, src_ld, perm_tok, it.g, it.r0, it.n,
                                             it.row0, it.wt, dst, dst_ld, lds, &wq);
  }
}

// ---- host side -------------------------------------------------------------------------------
// Upper bound of the tile-list length: rows / wide full tiles, plus per group at most one
// partial wide tile or (wide - narrow) / narrow narrow tiles.
int tiled_max_tiles(int64_t rows, int groups) {
  static_assert(Wide::kWT % Narrow::kWT == 0, "narrow tiles divide wide ones");
  return static_cast<int>(rows / Wide::kWT) + groups * ((Wide::kWT - Narrow::kWT) / Narrow::kWT) + 1;
}

// ---- tiled weight layout -----------------------------------------------------------------
// One k-tile block = kWM weight rows x kBK bf16 of one weight tile, 2048 16-byte slots in the
// LDS order of the ring: slot s holds chunk (s % 8) ^ f(s / 8) of tile row s / 8 (the swizzle
// of the tile shapes). Tile rows follow tile_product: for gate_up, 32-row blocks alternate the
// gate and the up rows of 32 channels (tile wt: channels 128 wt ..); for down, tile wt holds
// output rows 256 wt ... Blocks run k-tile by k-tile within a tile, tile by tile within a
// group. One thread per slot; reads are 16-byte row chunks, writes are contiguous.
static_assert(Wide::kBK == Narrow::kBK && Wide::kBK == Tiny::kBK, "one tiled layout for every shape");
static_assert(Wide::kRows == kWM && Narrow::kRows == kWM && Tiny::kRows == kWM, "kWM-row weight tiles");
constexpr int kPackSlots = kWM * Wide::kChunks;    // 16-byte slots per k-tile block
__global__ __launch_bounds__(256) void pack_tiled_kernel(const uint16_t* __restrict__ gate,
                                                         const uint16_t* __restrict__ up,
                                                         int64_t group_stride, int64_t total,
                                                         int tiles, int K, int gate_up,
                                                         uint16_t* __restrict__ dst) {
  const int nk = K / Wide::kBK;
  for (int64_t i = blockIdx.x * int64_t{256} + threadIdx.x; i < total;
       i += int64_t{256} * gridDim.x) {
    const int slot = static_cast<int>(i % kPackSlots);
    const int64_t blk = i / kPackSlots;
    const int kt = static_cast<int>(blk % nk);
    const int wt = static_cast<int>((blk / nk) % tiles);
    const int64_t grp = blk / nk / tiles;
    const int r = slot / Wide::kChunks;
    const int j = (slot % Wide::kChunks) ^ ((r >> Wide::kSwzShift) & (Wide::kChunks - 1));
    const uint16_t* srow;
    if (gate_up) {
      const int b = r >> 5;
      const int ch = wt * (kWM / 2) + 32 * (b >> 1) + (r & 31);
      srow = ((b & 1) ? up : gate) + grp * group_stride + static_cast<int64_t>(ch) * K;
    } else {
      srow = gate + grp * group_stride + static_cast<int64_t>(wt * kWM + r) * K;
    }
    *reinterpret_cast<u32x4*>(dst + i * 8) = ld16(srow + kt * Wide::kBK + 8 * j);
  }
}

hipError_t launch_pack_tiled(const uint16_t* gate, const uint16_t* up, int64_t group_stride,
                             int groups, int C, int K, bool gate_up, uint16_t* dst,
                             hipStream_t s) {
  const int rows_per_tile = gate_up ? kWM / 2 : kWM;
  const int tiles = C / rows_per_tile;
  const int64_t total = static_cast<int64_t>(groups) * tiles * (K / Wide::kBK) * kPackSlots;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  pack_tiled_kernel<<<static_cast<unsigned>(blocks < 65536 ? blocks : 65536), 256, 0, s>>>(
      gate, up, group_stride, total, tiles, K, gate_up ? 1 : 0, dst);
  return hipGetLastError();
}

bool tiled_supported(const GroupWeights& gw) {
  constexpr int kBKmax = Wide::kBK > Narrow::kBK ? Wide::kBK : Narrow::kBK;
  return gw.H % kWM == 0 && gw.H % kBKmax == 0 && gw.I % (kWM / 2) == 0 &&
         (gw.Is == 0 || gw.Is % (kWM / 2) == 0) && gw.I % kBKmax == 0 &&
         (gw.Is == 0 || gw.Is % kBKmax == 0) && gw.I < (1 << 20) && gw.E < (1 << 16) - 1;
}

bool tiled_offsets_fit(const GroupWeights& gw, int64_t T, int k) {
  return bf16_tiled_offsets_fit(T, k, gw.H, gw.I > gw.Is ? gw.I : gw.Is);
}

// Workgroups of a bf16 GEMM launch: one per possible item; the per-XCD rounding of the two item
// ranges adds at most 16 slots.
static int item_grid(int max_tiles, int n_wtiles) {
  return static_cast<int>(round8(static_cast<int64_t>(max_tiles) * n_wtiles + 16));
}
static int gate_up_wtiles(int I, int Is) { return (I > Is ? I : Is) / (kWM / 2); }
static int down_wtiles(int H) { return H / kWM; }

int64_t tiled_list_bytes(int max_tiles, int I, int Is, int H) {
  const int64_t slots = item_grid(max_tiles, gate_up_wtiles(I, Is)) +
                        item_grid(max_tiles, down_wtiles(H));
  return table_base(max_tiles) * 4 + slots * 16 + kQueueInts * 4;       // + the work queues
}

int tiled_grid(const GroupWeights& gw, int max_tiles, bool gate_up) {
  return item_grid(max_tiles, gate_up ? gate_up_wtiles(gw.I, gw.Is) : down_wtiles(gw.H));
}

const u32x4* tiled_table(const GroupWeights& gw, const int32_t* tiles, int max_tiles,
                         bool gate_up) {
  const auto* t = reinterpret_cast<const u32x4*>(tiles + table_base(max_tiles));
  return gate_up ? t : t + tiled_grid(gw, max_tiles, true);
}

// Workgroups that build a tile list with `entries` dispatch-table entries.
static int build_blocks(int max_tiles, int entries) {
  if (max_tiles > kLdsListEntries) return 1;   // a list past kLdsListEntries is read back from memory
  const int blocks = (entries + kBuildEntriesPerBlock - 1) / kBuildEntriesPerBlock;
  return blocks < 1 ? 1 : (blocks > kBuildBlocks ? kBuildBlocks : blocks);
}

hipError_t launch_build_tiles(const int32_t* counts, const int32_t* offsets, const GroupWeights& gw,
                              bool shared, int64_t T, int max_tiles, int32_t* tiles,
                              hipStream_t s) {
  const int grid_gu = tiled_grid(gw, max_tiles, true), grid_dn = tiled_grid(gw, max_tiles, false);
  build_tiles_kernel<<<build_blocks(max_tiles, grid_gu + grid_dn), 1024, 0, s>>>(counts, offsets, gw.E, shared ? 1 : 0,
                                             static_cast<int>(T), gw.sh_row0, max_tiles,
                                             Wide::kWT, Narrow::kWT, Tiny::kWT, gw.I, gw.Is, gw.H,
                                             grid_gu, grid_dn, tiles);
  return hipGetLastError();
}

// CUs of the current device, rounded down to a multiple of 8 (every XCD the same number).
// Looked up once per device; host threads that race on the first lookup store the same value.
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cus[kMaxDevices];   // per device (0: not yet looked up)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    c = n >= 8 ? n / 8 * 8 : 8;
    cus[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

// The persistent gate_up launch (one workgroup per CU) takes over from this many table entries
// per CU: with fewer items per CU the in-order hardware dispatch leaves little idle and the
// persistent loop's per-item queue work costs more than it saves (Qwen3-30B-A3B T=1024: 3.8
// entries per CU, 2-5 us slower).

hipError_t launch_gate_up_tiled(const GroupWeights& gw, const void* x, const int32_t* perm_tok,
                                const int32_t* tiles, int max_tiles, int64_t T, int act_ld,
                                void* act, hipStream_t s) {
  const int grid = tiled_grid(gw, max_tiles, true), cus = device_cus();
  const auto* xx = static_cast<const uint16_t*>(x);
  const u32x4* table = tiled_table(gw, tiles, max_tiles, true);
  auto* out = static_cast<uint16_t*>(act);
  if (grid >= kPersistentMinEntriesPerCu * cus) {
    int32_t* q = queue_base(const_cast<int32_t*>(tiles), max_tiles, grid,
                            tiled_grid(gw, max_tiles, false));
    tiled_persistent_kernel<kGateUp><<<cus, kThreads, 0, s>>>(gw, xx, gw.H, perm_tok, table,
                                                              grid / 8, q, out, act_ld);
  } else {
    tiled_kernel<kGateUp><<<grid, kThreads, 0, s>>>(gw, xx, gw.H, perm_tok, table,
                                                    static_cast<int>(T), out, act_ld);
  }
  return hipGetLastError();
}

hipError_t launch_down_tiled(const GroupWeights& gw, const void* act, int act_ld,
                             const int32_t* tiles, int max_tiles, int64_t T, void* out,
                             hipStream_t s) {
  tiled_kernel<kDown><<<tiled_grid(gw, max_tiles, false), kThreads, 0, s>>>(
      gw, static_cast<const uint16_t*>(act), act_ld, nullptr,
      tiled_table(gw, tiles, max_tiles, false), static_cast<int>(T),
      static_cast<uint16_t*>(out), gw.H);
  return hipGetLastError();
}

bool tiled_router_supported(int E, int H) { return H % RouterShape::kBK == 0 && E >= 1; }

template <class S>
static hipError_t launch_router_shape(const GroupWeights& gw, const void* x, int64_t T, void* logits,
                                      hipStream_t s) {
  const int n_wtiles = (gw.E + S::kRows - 1) / S::kRows;
  const int64_t n_ttiles = (T + S::kWT - 1) / S::kWT;
  router_tiled_kernel<S><<<round8(n_ttiles * n_wtiles), kThreads, 0, s>>>(
      gw, static_cast<const uint16_t*>(x), static_cast<int>(T), n_wtiles,
      static_cast<uint16_t*>(logits));
  return hipGetLastError();
}

bool router_route_supported(int E, int H, int k) {
  return E <= RouterShape128::kRows && tiled_router_supported(E, H) && k >= 1 && k <= kRouteMaxK &&
         k <= E;
}

int64_t router_route_chunks(int64_t T, int k) {
  return (T + RouterShape128::kWT - 1) / RouterShape128::kWT * k;
}

static int bits_of(int E) {
  int n = 0;
  while ((1 << n) < E) ++n;
  return n;
}

// Splits of the router's k range (router_partial_kernel): doubled while the blocks' workgroups
// leave CUs idle, each split keeping at least kSplitMinKTiles k-tiles, and the partial sums
// fitting part_bytes. 1: the one-launch router_route_kernel. The selection workgroup reads
// splits x 32 KB of sums, so more splits move bytes from the first launch's workgroups to the
// second's: Qwen3-30B-A3B router stage at T=1024 20.3 (one launch) / 16.3 (4 splits) / 19.0 us
// (8 splits), T=2048 24.2 / 18.8 / 21.8 us; at T=4096 4 splits 19.9 against 2 splits 21.7 us.
constexpr int kRouteMaxSplits = 4;
constexpr int kSplitMinKTiles = 4;
static int router_route_splits(int64_t T, int H, size_t part_bytes) {
  using S = RouterShape128;
  const int64_t nb = (T + S::kWT - 1) / S::kWT;
  const int nkt = H / S::kBK;
  int splits = 1;
  while (splits < kRouteMaxSplits && nb * splits < device_cus() && nkt % (2 * splits) == 0 &&
         nkt / (2 * splits) >= kSplitMinKTiles &&
         static_cast<size_t>(nb * 2 * splits) * kPartialFloats<S> * 4 <= part_bytes)
    splits *= 2;
  return splits;
}

hipError_t launch_router_route(const void* x, const void* wg, const float* bias, const void* w_sg,
                               int64_t T, int E, int H, int k, void* logits, int32_t* idx,
                               void* topw, float* sgate, int32_t* hist, int32_t* lrank,
                               void* part, size_t part_bytes, hipStream_t s) {
  GroupWeights gw{};
  gw.gate_up = wg;
  gw.E = E;
  gw.H = H;
  const int nb = static_cast<int>((T + RouterShape128::kWT - 1) / RouterShape128::kWT);
  const auto* xx = static_cast<const uint16_t*>(x);
  const auto* ws = static_cast<const uint16_t*>(w_sg);
  auto* lg = static_cast<uint16_t*>(logits);
  auto* tw = static_cast<uint16_t*>(topw);
  const int Ti = static_cast<int>(T), nbits = bits_of(E);
  const int splits = router_route_splits(T, H, part_bytes);
  if (splits == 1) {
    if (E <= 64)
      router_route_kernel<8><<<round8(nb), kThreads, 0, s>>>(gw, xx, Ti, bias, ws, k, nbits, nb, lg,
                                                             idx, tw, sgate, hist, lrank);
    else
      router_route_kernel<16><<<round8(nb), kThreads, 0, s>>>(gw, xx, Ti, bias, ws, k, nbits, nb,
                                                              lg, idx, tw, sgate, hist, lrank);
    return hipGetLastError();
  }
  auto* pt = static_cast<float*>(part);
  router_partial_kernel<<<round8(static_cast<int64_t>(nb) * splits), kThreads, 0, s>>>(
      gw, xx, Ti, nb, splits, pt);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
#define LBMOE_SELECT(EPG, SPLITS)                                                               \
  router_select_kernel<EPG, SPLITS><<<round8(nb), kThreads, 0, s>>>(gw, xx, Ti, pt, bias, ws, k, \
                                                                    nbits, nb, lg, idx, tw,     \
                                                                    sgate, hist, lrank)
  static_assert(kRouteMaxSplits == 4, "a selection kernel per split count");
  if (E <= 64) {
    if (splits == 2) LBMOE_SELECT(8, 2);
    else LBMOE_SELECT(8, 4);
  } else {
    if (splits == 2) LBMOE_SELECT(16, 2);
    else LBMOE_SELECT(16, 4);
  }
#undef LBMOE_SELECT
  return hipGetLastError();
}

hipError_t launch_scatter_build(const int32_t* idx, int64_t T, int k, const int32_t* base,
                                const int32_t* counts, const int32_t* lrank, int32_t* offsets,
                                int32_t* perm_tok, int32_t* perm_slot, int32_t* inv,
                                const GroupWeights& gw, bool shared, int max_tiles,
                                int32_t* tiles, hipStream_t s) {
  const int nb = static_cast<int>((T + RouterShape128::kWT - 1) / RouterShape128::kWT);
  const int n_scatter = (nb * k + 15) / 16;
  const int grid_gu = tiled_grid(gw, max_tiles, true), grid_dn = tiled_grid(gw, max_tiles, false);
  const int blocks = build_blocks(max_tiles, grid_gu + grid_dn);
  scatter_build_kernel<<<n_scatter + blocks, 1024, 0, s>>>(
      idx, static_cast<int>(T), k, nb, base, counts, lrank, offsets, perm_tok, perm_slot, inv,
      n_scatter, gw.E, shared ? 1 : 0, gw.sh_row0, max_tiles, Wide::kWT, Narrow::kWT, Tiny::kWT,
      gw.I, gw.Is, gw.H, grid_gu, grid_dn, tiles);
  return hipGetLastError();
}

hipError_t launch_perm_scatter_build(const void* idx, int idx_bytes, int64_t T, int k,
                                     const int32_t* base, const int32_t* counts,
                                     const int32_t* lrank, int32_t* offsets, int32_t* perm_tok,
                                     int32_t* perm_slot, int32_t* inv, const GroupWeights& gw,
                                     bool shared, int max_tiles, int32_t* tiles, hipStream_t s) {
  const int V = static_cast<int>(T * k);
  const int nblk = static_cast<int>(perm_blocks(V));
  const int n_scatter = nblk;
  const int grid_gu = tiled_grid(gw, max_tiles, true), grid_dn = tiled_grid(gw, max_tiles, false);
  const int blocks = build_blocks(max_tiles, grid_gu + grid_dn);
#define LBMOE_PSB(IB)                                                                           \
  perm_scatter_build_kernel<IB><<<n_scatter + blocks, 1024, 0, s>>>(                           \
      idx, static_cast<int>(T), k, V, nblk, base, counts, lrank, offsets, perm_tok, perm_slot, \
      inv, n_scatter, gw.E, shared ? 1 : 0, gw.sh_row0, max_tiles, Wide::kWT, Narrow::kWT,     \
      Tiny::kWT, gw.I, gw.Is, gw.H, grid_gu, grid_dn, tiles)
  if (idx_bytes == 8) LBMOE_PSB(8);
  else LBMOE_PSB(4);
#undef LBMOE_PSB
  return hipGetLastError();
}

hipError_t launch_router_logits_tiled(const void* x, const void* wg, int64_t T, int E, int H,
                                      void* logits, hipStream_t s) {
  GroupWeights gw{};
  gw.gate_up = wg;
  gw.E = E;
  gw.H = H;
  if (E <= RouterShape128::kRows) return launch_router_shape<RouterShape128>(gw, x, T, logits, s);
  const int64_t tall = (T + RouterShapeTall::kWT - 1) / RouterShapeTall::kWT *
                       ((E + RouterShapeTall::kRows - 1) / RouterShapeTall::kRows);
  if (tall >= kRouterTallMinWorkgroups)
    return launch_router_shape<RouterShapeTall>(gw, x, T, logits, s);
  // a workgroup of 256 x 64 tiles is bound by its own MFMA work: while those leave CUs idle,
  // 128 x 64 tiles give twice the workgroups
  const int64_t wide = (T + RouterShape::kWT - 1) / RouterShape::kWT *
                       ((E + RouterShape::kRows - 1) / RouterShape::kRows);
  if (wide < device_cus()) return launch_router_shape<RouterShape128>(gw, x, T, logits, s);
  return launch_router_shape<RouterShape>(gw, x, T, logits, s);
}

}  // namespace lbmoe
