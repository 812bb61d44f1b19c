// Host-side internals of liblbmoe: workspace layout and kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/lbmoe.h"

namespace lbmoe {

// Permutations of at most kPermSingle entries run in one workgroup; larger ones in chunks of
// kPermChunk entries, one wave per chunk.
constexpr int kPermSingle = 1024;
// Batches up to this many tokens (4 for E > 128) route and permute in one kernel
// (launch_route_perm_small).
constexpr int64_t kSmallRouteTokens = 16;
constexpr int kPermChunk = 256;

inline int64_t perm_blocks(int64_t V) { return (V + kPermChunk - 1) / kPermChunk; }

enum Region {
  R_LOGITS = 0, R_IDX, R_TOPW, R_SGATE, R_COUNTS, R_OFFSETS, R_PERM_TOK, R_PERM_SLOT, R_INV,
  R_ACT, R_OUT, R_XN,
  // private regions (not exposed through lbmoe_workspace_region)
  R_HIST, R_BASE, R_LRANK, R_TILES, R_XQ, R_XS, R_ACTQ, R_ACTS,
  R_COUNT_
};
constexpr int kPublicRegions = R_XN + 1;

struct WsLayout {
  size_t off[R_COUNT_];
  size_t bytes[R_COUNT_];
  size_t total;
};

WsLayout ws_layout(const lbmoe_layer& L, int64_t T);
// Layout of the permutation scratch (hist, base, lrank) alone.
void perm_scratch_layout(int64_t T, int k, int E, size_t* hist_off, size_t* base_off,
                         size_t* lrank_off, size_t* total);

// Per-group view of the expert weights for kernels. Groups 0..E-1 are the routed experts
// (rows offsets[g] .. offsets[g]+counts[g]-1 of the permuted arrays); group E is the shared
// expert, which takes all T tokens in order at rows sh_row0 .. sh_row0+T-1. A launch covers
// groups g0 .. g0+groups-1.
struct GroupWeights {
  const void* gate_up;      // [E,2I,H]
  const void* down;         // [E,H,I]
  const float* gate_up_scale;
  const float* down_scale;
  const void* sh_gate;      // [Is,H]
  const void* sh_up;        // [Is,H]
  const void* sh_down;      // [H,Is]
  const float* sh_gate_scale;
  const float* sh_up_scale;
  const float* sh_down_scale;
  // optional bf16 copies in the LDS-tiled GEMMs' tiled layout (pack_tiled_kernel), or null
  const void* gate_up_tiled;     // [E][I/128][H/64][256 x 64]
  const void* down_tiled;        // [E][H/256][I/64][256 x 64]
  const void* sh_gate_up_tiled;  // [Is/128][H/64][256 x 64]
  const void* sh_down_tiled;     // [H/256][Is/64][256 x 64]
  int E, H, I, Is;
  int g0, groups;
  int sh_row0;
  // > 0: the weight-streaming GEMMs give routed experts only this many rows of workgroups, row
  // y serving the y-th expert that received tokens (at most T*k of them exist), instead of one
  // row per expert; for small batches most experts receive none.
  int hit_rows;
};

// Grids of the weight-streaming GEMMs: the first rows of workgroups serve the routed groups,
// row y group g0 + y (or, with hit_rows, the y-th routed expert with tokens). The shared
// expert (the last group, when the launch has it) takes all T tokens, which one workgroup
// would walk pass after pass; it gets shared_extra more rows of workgroups after the routed
// ones, and slice s of its nslices takes passes s, s + nslices, ...
struct GroupSlice {
  int g, slice, nslices;   // g < 0: no group for this row
};

// The y-th expert (ascending) with counts[e] > 0 among E <= 1024, or -1; wave-uniform.
__device__ __forceinline__ int nth_hit(const int32_t* __restrict__ counts, int E, int y) {
  const int lane = threadIdx.x & 63;
  int c[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = counts[min(i * 64 + lane, E - 1)];   // all loads in flight
  int base = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint64_t m = __ballot(i * 64 + lane < E && c[i] > 0);
    const int cnt = __popcll(m);
    if (y < base + cnt) {
      const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
      const uint64_t sel = __ballot(((m >> lane) & 1) != 0 && below == y - base);
      return i * 64 + __ffsll(static_cast<unsigned long long>(sel)) - 1;
    }
    base += cnt;
  }
  return -1;
}

__host__ __device__ inline int routed_rows(const GroupWeights& gw) {
  const int has_shared = gw.g0 + gw.groups > gw.E ? 1 : 0;
  return gw.hit_rows > 0 ? gw.hit_rows : gw.groups - has_shared;
}
// Rows of workgroups of a weight-streaming GEMM launch before the shared expert's extra rows.
inline int grid_groups(const GroupWeights& gw) {
  return routed_rows(gw) + (gw.g0 + gw.groups > gw.E ? 1 : 0);
}

__device__ __forceinline__ GroupSlice group_slice(const GroupWeights& gw, int shared_extra,
                                                  const int32_t* __restrict__ counts) {
  const int y = blockIdx.y, rows = routed_rows(gw);
  if (y < rows) return {gw.hit_rows > 0 ? nth_hit(counts, gw.E, y) : gw.g0 + y, 0, 1};
  return {gw.E, y - rows, shared_extra + 1};
}
constexpr int kMaxSharedSlices = 16;
// Extra workgroup rows for the shared expert at tokens_per_pass tokens per pass.
inline int shared_extra_rows(const GroupWeights& gw, int64_t T, int tokens_per_pass) {
  if (gw.g0 + gw.groups <= gw.E) return 0;
  const int64_t passes = (T + tokens_per_pass - 1) / tokens_per_pass;
  return static_cast<int>((passes < kMaxSharedSlices ? passes : kMaxSharedSlices) - (passes > 0));
}

// ---- launchers (each returns hipError_t of the launch) ----------------------------------
hipError_t launch_router_logits(const void* x, const void* wg, int64_t T, int E, int H,
                                void* logits, hipStream_t s);
// Residual add + RMSNorm of the decoder layer ahead of the block, then the router logits of
// its output: x_out = the block's input, res_out = the new residual (fused into the router
// for decode-sized T).
hipError_t launch_add_rmsnorm_router(const void* hidden, const void* residual, const void* norm_w,
                                     float eps, const void* wg, int64_t T, int E, int H,
                                     void* logits, void* x_out, void* res_out, hipStream_t s);
// xq, xs (fp8 layers, with sgate): x's e4m3 codes and group scales, written with the shared
// gate's loads of x (quant_groups_kernel's layout), so the layer needs no separate pass.
hipError_t launch_route_topk(const void* logits, const float* bias, const void* x,
                             const void* w_sg, int64_t T, int E, int H, int k, void* idx,
                             int idx_bytes, void* topw, float* sgate, hipStream_t s,
                             void* xq = nullptr, float* xs = nullptr);
bool route_perm_small_supported(int64_t T, int k, int E);
hipError_t launch_route_perm_small(const void* logits, const float* bias, const void* x,
                                   const void* w_sg, int64_t T, int E, int H, int k, int32_t* idx,
                                   void* topw, float* sgate, int32_t* counts, int32_t* offsets,
                                   int32_t* perm_tok, int32_t* perm_slot, int32_t* inv,
                                   hipStream_t s);
hipError_t launch_permute(const void* idx, int idx_bytes, int64_t T, int k, int E,
                          bool shared_rows, int32_t* counts, int32_t* offsets,
                          int32_t* perm_tok, int32_t* perm_slot, int32_t* inv,
                          int32_t* hist, int32_t* base, int32_t* lrank, hipStream_t s);
hipError_t launch_gate_up_bf16(const GroupWeights& gw, const void* x, const int32_t* counts,
                               const int32_t* offsets, const int32_t* perm_tok, int64_t T,
                               int k, int act_ld, void* act, hipStream_t s);
// Batches of at most kInlineRouteTokens tokens (and T*k <= kInlineRouteEntries) skip the
// route and permutation kernels on the bf16 decode path: every gate_up workgroup selects the
// batch's experts from the logits itself (launch_gate_up_bf16_routed) and derives its own
// group's rows, and the workgroups of the first channel block store the routing outputs.
constexpr int64_t kInlineRouteTokens = 4;
constexpr int kInlineRouteEntries = 64;
bool inline_route_supported(int64_t T, int k, int E);
// What the routed gate_up launch reads and writes besides the GEMM operands: the route's
// inputs (logits, the optional bias and shared-expert gate weight) and the outputs of the
// route and permutation kernels it replaces.
struct SmallRoute {
  const uint16_t* logits;
  const float* bias;
  const uint16_t* w_sg;
  int k;
  int32_t* idx;
  uint16_t* topw;
  float* sgate;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm_tok;
  int32_t* perm_slot;
  int32_t* inv;
};
hipError_t launch_gate_up_bf16_routed(const GroupWeights& gw, const void* x, const SmallRoute& rt,
                                      int64_t T, int act_ld, void* act, hipStream_t s);
// Decode batches whose every expert can receive tokens (T*k >= E, so each routed workgroup row
// is one expert) skip the permutation kernel: each gate_up workgroup derives its expert's rows
// from the selected experts (launch_gate_up_bf16_perm), channel block 0 writes them out, and
// workgroup (0, 0) the counts and offsets. At most kFusedPermTokens tokens; the expert ids must
// lie in [0, E) (the route's own output).
constexpr int64_t kFusedPermTokens = 256;
struct PermOut {
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm_tok;
  int32_t* perm_slot;
  int32_t* inv;
};
bool gate_up_perm_supported(const GroupWeights& gw, int64_t T, int k);
hipError_t launch_gate_up_bf16_perm(const GroupWeights& gw, const void* x, const int32_t* idx,
                                    const PermOut& po, int64_t T, int k, int act_ld, void* act,
                                    hipStream_t s);
hipError_t launch_down_bf16(const GroupWeights& gw, const void* act, int act_ld,
                            const int32_t* counts, const int32_t* offsets, int64_t T, int k,
                            void* out, hipStream_t s);
// Batches of at most kFusedDownTokens tokens (bf16, weight streaming) run the down GEMM and
// the combine as one kernel (launch_down_combine_small); the expert_out region is then not
// written. Columns per workgroup and the LDS bound on entries (T*k + T).
constexpr int64_t kFusedDownTokens = 4;
constexpr int kFusedCols = 8;
constexpr int kFusedDownEntries = 66;
bool down_combine_small_supported(const GroupWeights& gw, int64_t T, int k);
hipError_t launch_down_combine_small(const GroupWeights& gw, const void* act, int act_ld,
                                     const int32_t* idx, const int32_t* inv, const void* topw,
                                     const float* sgate, int64_t T, int k, bool shared, void* y,
                                     hipStream_t s);
hipError_t launch_combine(const void* out_rows, const int32_t* inv, const void* topw,
                          const float* sgate, int64_t T, int k, int H, bool shared,
                          void* y, hipStream_t s);
// LDS-tiled grouped GEMMs (prefill-sized batches) over a tile list of wide, narrow and tiny
// token tiles, with one dispatch table per GEMM launch (bf16 and fp8 kernels share both).
// Words behind a tile list's entries: count, wide count.
constexpr int kTileListTail = 2;
int tiled_max_tiles(int64_t rows, int groups);  // rows = routed + shared
// Bytes of a tile list with max_tiles entries and the dispatch tables of both GEMMs.
int64_t tiled_list_bytes(int max_tiles, int I, int Is, int H);
bool tiled_supported(const GroupWeights& gw);
// Whether every byte offset of the bf16 tiled GEMMs' buffer copies stays below 2^31 for a call
// of T tokens (x, the act rows of the routed and shared experts, one expert's weight matrix).
bool tiled_offsets_fit(const GroupWeights& gw, int64_t T, int k);
// CUs of the current device, rounded down to a multiple of 8 (every XCD the same number).
int device_cus();
// The persistent gate_up launches (one workgroup per CU) take over from this many table entries
// per CU: with fewer items per CU the in-order hardware dispatch leaves little idle and the
// persistent loop's per-item queue work costs more than it saves (bf16 Qwen3-30B-A3B T=1024:
// 3.8 entries per CU, 2-5 us slower).
constexpr int kPersistentMinEntriesPerCu = 6;
// rows = routed + shared rows of the call
bool tiled_fp8_supported(const GroupWeights& gw, int64_t T, int64_t rows);
hipError_t launch_build_tiles(const int32_t* counts, const int32_t* offsets, const GroupWeights& gw,
                              bool shared, int64_t T, int max_tiles, int32_t* tiles,
                              hipStream_t s);
hipError_t launch_gate_up_tiled(const GroupWeights& gw, const void* x, const int32_t* perm_tok,
                                const int32_t* tiles, int max_tiles, int64_t T, int act_ld,
                                void* act, hipStream_t s);
// Writes the tiled layout of bf16 weights for the LDS-tiled GEMMs. gate_up: gate and up are
// [C, K] row blocks (C channels) of `groups` groups, group_stride elements apart, written as
// [groups][C/128][K/64] blocks; otherwise w [C, K] (C output rows) as [groups][C/256][K/64].
// dst holds as many elements as the source tensors.
hipError_t launch_pack_tiled(const uint16_t* gate, const uint16_t* up, int64_t group_stride,
                             int groups, int C, int K, bool gate_up, uint16_t* dst,
                             hipStream_t s);
hipError_t launch_down_tiled(const GroupWeights& gw, const void* act, int act_ld,
                             const int32_t* tiles, int max_tiles, int64_t T, void* out,
                             hipStream_t s);
// fp8: gate_up writes the quantised act (e4m3 codes, act_ld bytes per row, and per (row, 128)
// scales) that down reads.
hipError_t launch_gate_up_tiled_fp8(const GroupWeights& gw, const void* xq, const float* xs,
                                    const int32_t* perm_tok, const int32_t* tiles, int max_tiles,
                                    int act_ld, void* actq, float* acts, hipStream_t s);
hipError_t launch_down_tiled_fp8(const GroupWeights& gw, const void* actq, const float* acts,
                                 int act_ld, const int32_t* tiles, int max_tiles, void* out,
                                 hipStream_t s);
bool tiled_router_supported(int E, int H);
// whether launch_router_logits runs the LDS-tiled router for this batch
bool router_is_tiled(int64_t T, int E, int H);
// Router logits + selection + the permutation's count pass in one launch (E <= 128), then the
// per-expert scan (launch_perm_scan over router_route_chunks(T, k) chunks) and the scatter with
// the tile list (launch_scatter_build).
bool router_route_supported(int E, int H, int k);
int64_t router_route_chunks(int64_t T, int k);
// part: scratch for the k-split partial sums (part_bytes of it; with too little the router runs
// as one launch)
hipError_t launch_router_route(const void* x, const void* wg, const float* bias, const void* w_sg,
                               int64_t T, int E, int H, int k, void* logits, int32_t* idx,
                               void* topw, float* sgate, int32_t* hist, int32_t* lrank,
                               void* part, size_t part_bytes, hipStream_t s);
hipError_t launch_perm_scan(const int32_t* hist, int nchunks, int E, int32_t* base,
                            int32_t* totals, hipStream_t s);
// The chunked permutation of launch_permute as two steps, for the prefill GEMMs: the count
// and scan passes (perm_count, perm_expert_scan: hist, base, lrank, counts), then the scatter
// with the GEMMs' tile list in one launch. perm_chunked: whether launch_permute would chunk a
// batch of V entries (otherwise it permutes in one workgroup).
bool perm_chunked(int64_t V, int E);
hipError_t launch_perm_count_scan(const void* idx, int idx_bytes, int64_t T, int k, int E,
                                  int32_t* hist, int32_t* base, int32_t* lrank, int32_t* counts,
                                  hipStream_t s);
hipError_t launch_perm_scatter_build(const void* idx, int idx_bytes, int64_t T, int k,
                                     const int32_t* base, const int32_t* counts,
                                     const int32_t* lrank, int32_t* offsets, int32_t* perm_tok,
                                     int32_t* perm_slot, int32_t* inv, const GroupWeights& gw,
                                     bool shared, int max_tiles, int32_t* tiles, hipStream_t s);
hipError_t launch_scatter_build(const int32_t* idx, int64_t T, int k, const int32_t* base,
                                const int32_t* counts, const int32_t* lrank, int32_t* offsets,
                                int32_t* perm_tok, int32_t* perm_slot, int32_t* inv,
                                const GroupWeights& gw, bool shared, int max_tiles,
                                int32_t* tiles, hipStream_t s);
hipError_t launch_router_logits_tiled(const void* x, const void* wg, int64_t T, int E, int H,
                                      void* logits, hipStream_t s);
hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t s);
hipError_t launch_quant_blocks_fp8(const void* w, int64_t batch, int N, int K, void* q,
                                   float* scale, hipStream_t s);
hipError_t launch_quant_groups_fp8(const void* a, int64_t rows, int cols, int ld, void* q,
                                   float* scale, hipStream_t s);
hipError_t launch_gate_up_fp8(const GroupWeights& gw, const void* xq, const float* xs,
                              const int32_t* counts, const int32_t* offsets,
                              const int32_t* perm_tok, int64_t T, int k, int act_ld, void* act,
                              hipStream_t s);
hipError_t launch_down_fp8(const GroupWeights& gw, const void* actq, const float* acts,
                           int act_ld, const int32_t* counts, const int32_t* offsets,
                           int64_t T, int k, void* out, hipStream_t s);

}  // namespace lbmoe
