// Tile geometry and dispatch-table format shared by the LDS-tiled GEMMs (tiled_gemm.hip for
// bf16 operands, tiled_fp8.hip for e4m3 operands).
//
// A workgroup has kWaves waves (two per SIMD) and multiplies kWM weight rows (MFMA rows) by a
// tile of tokens (MFMA columns) of one group. Both operands move global -> LDS in k-tiles of
// 128 bytes per row (64 bf16 or 128 e4m3 values), as 16-byte chunks whose position within
// the LDS row is a row-dependent XOR of the chunk index, so that 16 consecutive rows of one
// chunk hit distinct bank groups.
#pragma once

#include "internal.hpp"
#include "tiled_common.hpp"

namespace lbmoe {

constexpr int kWaves = 8;                           // two waves per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kWM = 256;                            // weight rows per workgroup

// One token-tile shape: WAVES_M x (kWaves / WAVES_M) waves, each owning MT x NT units of 32
// weight rows x 32 tokens, k-tiles of BK bf16 (2 * BK bytes per row), STAGES LDS buffers of
// the weight operand and BSTAGES (STAGES or STAGES - 1) of the token operand. A symmetric ring
// interleaves the operands per stage; an asymmetric one keeps all weight stages first. The
// expert GEMMs use kRows = kWM weight rows; the router may use fewer.
template <int WAVES_M, int MT, int NT, int BK, int STAGES, int BSTAGES = STAGES>
struct TileShape {
  static constexpr int kRows = WAVES_M * MT * 32;             // weight rows per workgroup
  static constexpr int kWavesM = WAVES_M;
  static constexpr int kWavesN = kWaves / WAVES_M;
  static constexpr int kMT = MT;
  static constexpr int kNT = NT;
  static constexpr int kRW = MT * 32;                         // weight rows per wave
  static constexpr int kWT = kWavesN * NT * 32;               // tokens per workgroup
  static constexpr int kBK = BK;
  static constexpr int kStages = STAGES;
  static constexpr int kBStages = BSTAGES;
  static constexpr int kChunks = BK / 8;                      // 16-byte chunks per LDS row
  static constexpr int kRowsPerLoad = 64 / kChunks;           // rows one wave copy covers
  static constexpr int kALoads = kRows / kRowsPerLoad / kWaves;  // wave copies per stage (weights)
  static constexpr int kBLoads = kWT / kRowsPerLoad / kWaves;  // wave copies per stage (tokens)
  static constexpr int kLoads = kALoads + kBLoads;
  static constexpr int kStageU4 = (kRows + kWT) * kChunks;    // 16-byte slots per stage
  static constexpr int kAU4 = kRows * kChunks, kBU4 = kWT * kChunks;
  static constexpr bool kAsym = BSTAGES != STAGES;
  static constexpr int kRingU4 = kAsym ? STAGES * kAU4 + BSTAGES * kBU4 : STAGES * kStageU4;
  static_assert(!kAsym || BSTAGES + 1 == STAGES, "asymmetric ring: one more weight stage");
  static constexpr int a_off(int s) { return kAsym ? s * kAU4 : s * kStageU4; }
  static constexpr int b_off(int s) { return kAsym ? STAGES * kAU4 + s * kBU4 : s * kStageU4 + kAU4; }
  static constexpr int kKSteps = BK / 16;                     // bf16 MFMA k-steps per k-tile
  // Chunk j of row r lives at slot r*kChunks + (j ^ f(r)), f(r) = (r / (16/kChunks)) mod
  // kChunks: 16 consecutive rows then hit 16 distinct 16-byte bank groups for any fixed j.
  static constexpr int kSwzShift = kChunks == 4 ? 2 : 1;
  static_assert(kChunks == 4 || kChunks == 8, "BK must be 32 or 64");
  static_assert(kALoads * kRowsPerLoad * kWaves == kRows && kBLoads * kRowsPerLoad * kWaves == kWT,
                "copies must tile the stage");
  static_assert(kKSteps % 2 == 0, "the next k-tile's first fragments go to register buffer 0");
  static __device__ __forceinline__ int swz(int r, int j) {
    return r * kChunks + (j ^ ((r >> kSwzShift) & (kChunks - 1)));
  }
};

// Narrow and tiny token tiles carry these flags on their first row.
constexpr int32_t kNarrowFlag = 1 << 30;
constexpr int32_t kTinyFlag = 1 << 29;

// One dispatch-table entry (16 bytes, written by build_tiles_kernel): the work of one
// workgroup of a GEMM launch.
struct TileItem {
  int g;        // group (expert; E = shared expert); negative: no work
  int wt;       // weight tile
  int r0;       // first row of the token tile within the group
  bool narrow;  // narrow token tile
  bool tiny;    // tiny token tile (a group's last rows, at most a tiny tile's width)
  int row0;     // the group's first row in the expert-sorted rows
  int n;        // the group's row count
};
__device__ __forceinline__ TileItem decode_item(u32x4 ent) {
  TileItem it;
  const int gx = static_cast<int>(ent[0]);
  it.g = gx < 0 ? -1 : (gx & 0xffff);
  it.wt = gx >> 16;
  const int e = static_cast<int>(ent[1]);
  it.narrow = (e & kNarrowFlag) != 0;
  it.tiny = (e & kTinyFlag) != 0;
  it.r0 = e & (kTinyFlag - 1);
  it.row0 = static_cast<int>(ent[2]);
  it.n = static_cast<int>(ent[3]);
  return it;
}

// Output tile staged in LDS as row-major [token][column] bf16: 16-byte chunk c of staged row r
// sits at chunk c ^ (r mod kRowChunks), which spreads the rows of an accumulator write over
// distinct banks.
template <int kCols>
__device__ __forceinline__ int staged_slot(int r, int c) {
  constexpr int kRowChunks = kCols / 8;
  return r * kRowChunks + (c ^ (r & (kRowChunks - 1)));
}

// Stores staged rows r < min(kTokens, n - r0) to dst[row0 + r0 + r, c0 .. c0 + kCols) with
// 16-byte lanes, whole row segments at a time. NT: non-temporal stores, for output that only
// the combine reads back once (the down GEMMs: E=512 T=4096 down 256 -> 245 us, fp8 E=512
// T=16384 413 -> 405 us), so that it does not displace the operands the GEMM reuses.
template <int kCols, int kTokens, bool NT = false>
__device__ __forceinline__ void store_staged(const u32x4* __restrict__ st, uint16_t* __restrict__ dst,
                                             int dst_ld, int row0, int r0, int n, int c0) {
  constexpr int kRowChunks = kCols / 8;
  constexpr int kRowsPerPass = kThreads / kRowChunks;
  const int c = threadIdx.x % kRowChunks;
  for (int r = threadIdx.x / kRowChunks; r < kTokens; r += kRowsPerPass) {
    const int p = r0 + r;
    if (p >= n) break;
    u32x4* d = reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(row0 + p) * dst_ld + c0 + 8 * c);
    if constexpr (NT) __builtin_nontemporal_store(st[staged_slot<kCols>(r, c)], d);
    else *d = st[staged_slot<kCols>(r, c)];
  }
}

// Words of the tile list before the dispatch tables (entries, counts), rounded to 16 bytes.
__host__ __device__ constexpr int64_t table_base(int max_tiles) {
  return (2 * static_cast<int64_t>(max_tiles) + kTileListTail + 3) / 4 * 4;
}

// Work queues of the persistent gate_up launch, behind both dispatch tables: 8 counters (one per
// XCD, 64 ints apart so that they sit on different cache lines), then the 8 queue lengths.
constexpr int kQueueInts = 8 * 64 + 8;
__host__ __device__ inline int32_t* queue_base(int32_t* tiles, int max_tiles, int grid_gu,
                                               int grid_dn) {
  return tiles + table_base(max_tiles) + 4 * static_cast<int64_t>(grid_gu + grid_dn);
}

// Work queue of a persistent workgroup. XCD x's queue holds the dispatch-table entries
// table[j * 8 + x], j < its length (the items a launch of one workgroup per entry would run on
// that XCD, in the same order); its counter hands them out. A workgroup takes entries from its
// home XCD's queue and, once that is empty, from the others in turn, so the last items of a
// slow XCD spread over the chip.
struct WorkQueue {
  const u32x4* table;
  int slots;       // table entries per XCD
  int* q;          // counters q[x * 64], lengths q[8 * 64 + x]
  int home;        // this workgroup's XCD
  int tried;       // queues found empty so far
  int own_len;     // length of the home queue
};

// Next entry (thread 0 only), synchronously: a queue whose counter has reached its length is
// passed by with a load, otherwise an atomic takes an entry or finds the queue exhausted, so a
// workgroup makes at most (entries taken + idle entries + 8) atomics.
__device__ __forceinline__ u32x4 queue_fetch(WorkQueue& wq) {
  while (wq.tried < 8) {
    const int x = (wq.home + wq.tried) & 7;
    int* cnt = wq.q + x * 64;
    const int len = min(wq.q[8 * 64 + x], wq.slots);
    if (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < len) {
      const int j = atomicAdd(cnt, 1);
      if (j < len) {
        const u32x4 e = wq.table[j * 8 + x];
        if (static_cast<int>(e[0]) >= 0) return e;
        continue;                                  // an idle entry: the queue's next one
      }
    }
    ++wq.tried;
  }
  return u32x4{0xffffffffu, 0u, 0u, 0u};
}

// Host side: workgroups of a GEMM launch and its dispatch table within the tile list.
int tiled_grid(const GroupWeights& gw, int max_tiles, bool gate_up);
const u32x4* tiled_table(const GroupWeights& gw, const int32_t* tiles, int max_tiles,
                         bool gate_up);

}  // namespace lbmoe
