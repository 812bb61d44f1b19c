// Expert sort of the (token, slot) routing pairs.
//
// Restates the ordering of the reference's _forward_sparse (nanovllm/models/qwen3_5.py:823-833):
// experts ascending, and within an expert torch.where over the [k, T] mask, i.e. (slot, token)
// row-major. Entries are visited in slot-major order v = s*T + t, so a stable counting sort
// on the expert id yields exactly the key (expert, slot, token).
//
// Integer-only and deterministic:
//   count     one wave per chunk of kPermChunk entries: stable rank of every entry among the
//             chunk's entries of the same expert (64-lane ballot matching on the expert
//             bits), per-chunk histogram hist[e][chunk].
//   per-expert one wave per expert: exclusive scan of hist[e][*] -> base[e][chunk], total[e].
//   scatter   one wave per chunk: offsets[e] = exclusive scan of the totals (each workgroup
//             scans them itself), pos = offsets[e] + base[e][chunk] + rank -> perm_tok,
//             perm_slot, inv.
// Up to 2 * kPermSingle entries (4 * kPermSingle for E <= 512), i.e. decode-sized batches, run
// all of it in a single workgroup.
// Entries whose expert id lies outside [0, E) are left out of every list and get inv = -1.
#include "common.hpp"
#include "internal.hpp"
#include "route_token.hpp"

namespace lbmoe {

// Ranks one chunk's entries. Returns per-lane (expert, rank) for round r in e_out/rk_out.
// All expert ids of the chunk are loaded before the ranking so the loads overlap.
template <int IB, int ROUNDS>
__device__ __forceinline__ void rank_chunk(const void* idx, int T, int k, int E, int nbits,
                                           int V, int v0, int* run, int (&e_out)[ROUNDS],
                                           int (&rk_out)[ROUNDS]) {
  const int lane = lane_id();
  // unconditional loads (entries past V read entry V-1 and are masked): a load under a
  // condition would make the compiler wait for it before issuing the next; V >= 1 here
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    const int v = min(v0 + r * kWave + lane, V - 1);
    const int s = v / T;
    const int t = v - s * T;
    e_out[r] = load_expert<IB>(idx, static_cast<int64_t>(t) * k + s);
  }
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r)
    if (v0 + r * kWave + lane >= V) e_out[r] = -1;
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    const int e = e_out[r];
    const bool valid = (e >= 0) && (e < E);
    const uint64_t m = match_expert(valid ? e : 0, __ballot(valid), nbits);
    int rank = -1;
    if (valid) {
      const int before = run[e];                       // same address for the whole group
      rank = before + mask_rank(m);
      if (mask_rank(m) == 0) run[e] = before + __popcll(m);   // group leader
    }
    e_out[r] = valid ? e : -1;
    rk_out[r] = rank;
  }
}

constexpr int kRounds = kPermChunk / kWave;

template <int IB>
__global__ __launch_bounds__(64) void perm_count(const void* idx, int T, int k, int E,
                                                 int nbits, int V, int nblk, int32_t* hist,
                                                 int32_t* lrank) {
  __shared__ int run[1024];
  const int lane = lane_id();
  for (int e = lane; e < E; e += kWave) run[e] = 0;
  __syncthreads();
  const int b = blockIdx.x;
  int ee[kRounds], rk[kRounds];
  rank_chunk<IB, kRounds>(idx, T, k, E, nbits, V, b * kPermChunk, run, ee, rk);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int v = b * kPermChunk + r * kWave + lane;
    if (v < V) lrank[v] = rk[r];
  }
  __syncthreads();
  for (int e = lane; e < E; e += kWave) hist[static_cast<int64_t>(e) * nblk + b] = run[e];
}

// Per expert (one wave each): exclusive scan of its per-chunk counts, and its total.
__global__ __launch_bounds__(64) void perm_expert_scan(const int32_t* __restrict__ hist, int nblk,
                                                       int32_t* __restrict__ base,
                                                       int32_t* __restrict__ totals) {
  const int e = blockIdx.x, lane = lane_id();
  const int per = (nblk + kWave - 1) / kWave;
  const int lo = min(nblk, lane * per), hi = min(nblk, lo + per);
  const int32_t* h = hist + static_cast<int64_t>(e) * nblk;
  int local = 0;
  for (int b = lo; b < hi; ++b) local += h[b];
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  int run = incl - local;
  int32_t* bs = base + static_cast<int64_t>(e) * nblk;
  for (int b = lo; b < hi; ++b) {
    const int c = h[b];
    bs[b] = run;
    run += c;
  }
  if (lane == 63) totals[e] = incl;
}

// The same with the expert's counts held in registers: 256 threads, thread t taking chunks
// t * PER .. t * PER + PER - 1 (all loads in flight at once, read once), then a block scan.
// The one-wave form above walks up to nblk / 64 chunks per lane twice, load after load.
template <int PER>
__global__ __launch_bounds__(256) void perm_expert_scan_reg(const int32_t* __restrict__ hist,
                                                            int nblk, int32_t* __restrict__ base,
                                                            int32_t* __restrict__ totals) {
  __shared__ int wsum[4];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int32_t* h = hist + static_cast<int64_t>(e) * nblk;
  const int b0 = tid * PER;
  int v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = h[min(b0 + i, nblk - 1)];   // unconditional loads
  int local = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (b0 + i >= nblk) v[i] = 0;
    local += v[i];
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int c = wsum[w];
    before += w < wv ? c : 0;
    total += c;
  }
  int run = before + incl - local;
  int32_t* bs = base + static_cast<int64_t>(e) * nblk;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (b0 + i < nblk) bs[b0 + i] = run;
    run += v[i];
  }
  if (tid == 0) totals[e] = total;
}

// Per-expert exclusive scans of E x nblk chunk counts (hist) into base and totals.
static void launch_expert_scan(const int32_t* hist, int nblk, int E, int32_t* base,
                               int32_t* totals, hipStream_t s) {
  if (nblk <= 256) perm_expert_scan_reg<1><<<E, 256, 0, s>>>(hist, nblk, base, totals);
  else if (nblk <= 512) perm_expert_scan_reg<2><<<E, 256, 0, s>>>(hist, nblk, base, totals);
  else if (nblk <= 1024) perm_expert_scan_reg<4><<<E, 256, 0, s>>>(hist, nblk, base, totals);
  else if (nblk <= 2048) perm_expert_scan_reg<8><<<E, 256, 0, s>>>(hist, nblk, base, totals);
  else perm_expert_scan<<<E, 64, 0, s>>>(hist, nblk, base, totals);
}

// Each workgroup first scans the E expert totals itself (exclusive, into LDS), so no separate
// offsets pass runs between the per-expert scan and the scatter; workgroup 0 also stores the
// offsets (E + 1 entries) for the later stages.
template <int IB>
__global__ __launch_bounds__(64) void perm_scatter(const void* idx, int T, int k, int E, int V,
                                                   int nblk, const int32_t* base,
                                                   const int32_t* totals, int32_t* offsets,
                                                   const int32_t* lrank, int32_t* perm_tok,
                                                   int32_t* perm_slot, int32_t* inv) {
  __shared__ int s_off[1024];
  const int lane = lane_id();
  const int b = blockIdx.x;
  // every expert id first, unconditionally (entries past V read entry V-1, V >= 1 here)
  int ev[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int v = min(b * kPermChunk + r * kWave + lane, V - 1);
    const int s = v / T;
    ev[r] = load_expert<IB>(idx, static_cast<int64_t>(v - s * T) * k + s);
  }
  // lane l scans experts [l * per, (l + 1) * per), per <= 16 (E <= 1024)
  const int per = (E + kWave - 1) / kWave;
  const int lo = min(E, lane * per), hi = min(E, lo + per);
  int local = 0;
  for (int e = lo; e < hi; ++e) local += totals[e];
  int incl = local;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  int run = incl - local;
  for (int e = lo; e < hi; ++e) {
    s_off[e] = run;
    if (b == 0) offsets[e] = run;
    run += totals[e];
  }
  if (b == 0 && lane == kWave - 1) offsets[E] = incl;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int v = b * kPermChunk + r * kWave + lane;
    if (v >= V) break;
    const int s = v / T;
    const int t = v - s * T;
    const int e = ev[r];
    const int64_t ts = static_cast<int64_t>(t) * k + s;
    if (e < 0 || e >= E) {
      inv[ts] = -1;
      continue;
    }
    const int pos = s_off[e] + base[static_cast<int64_t>(e) * nblk + b] + lrank[v];
    perm_tok[pos] = t;
    perm_slot[pos] = s;
    inv[ts] = pos;
  }
}

// Whole permutation in one workgroup for decode-sized batches (V <= R * kPermSingle): thread
// tid takes entries v = r * kPermSingle + tid, r < R, so that "virtual wave" vw = v / 64 =
// r * (kPermSingle / 64) + wave covers 64 consecutive entries. Each virtual wave ranks its
// entries among equal experts (ballot match) and records its count per expert; one thread per
// expert then turns the counts into per-virtual-wave prefixes (in v order) and a total, a block
// scan of the totals gives the offsets, and every entry lands at offsets[e] + (entries of e in
// earlier virtual waves) + rank.
// The body, for a workgroup of kPermSingle threads that all call it (idx may point to LDS).
template <int IB, int R, int EMAX>
__device__ __forceinline__ void perm_single_body(const void* idx, int T, int k, int E, int nbits,
                                                 int V, int32_t* counts, int32_t* offsets,
                                                 int32_t* perm_tok, int32_t* perm_slot,
                                                 int32_t* inv) {
  constexpr int kW = kPermSingle / kWave;
  constexpr int kVW = kW * R;            // virtual waves
  __shared__ int cnt[kVW][EMAX];         // per virtual wave and expert: count, then prefix
  __shared__ int start[EMAX];
  __shared__ int wsum[kW];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  for (int i = tid; i < kVW * EMAX; i += kPermSingle) (&cnt[0][0])[i] = 0;
  int e[R], s[R], t[R], rank[R];
  bool valid[R];
  // unconditional loads (entries past V read entry V-1 and are masked); V = 0 reads nothing
#pragma unroll
  for (int r = 0; r < R; ++r) {
    e[r] = -1;
    s[r] = t[r] = 0;
  }
  if (V > 0) {                           // the same for every thread
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int v = min(r * kPermSingle + tid, V - 1);
      s[r] = v / T;
      t[r] = v - s[r] * T;
      e[r] = load_expert<IB>(idx, static_cast<int64_t>(t[r]) * k + s[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r * kPermSingle + tid >= V) e[r] = -1;
  }
  uint64_t m[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    valid[r] = (e[r] >= 0) && (e[r] < E);
    m[r] = match_expert(valid[r] ? e[r] : 0, __ballot(valid[r]), nbits);
    rank[r] = mask_rank(m[r]);
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (valid[r] && rank[r] == 0) cnt[r * kW + wave][e[r]] = __popcll(m[r]);
  __syncthreads();
  int total = 0;
  if (tid < E) {
    for (int w = 0; w < kVW; ++w) {
      const int c = cnt[w][tid];
      cnt[w][tid] = total;
      total += c;
    }
  }
  int incl = total;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wsum[w];
  const int excl = before + incl - total;
  if (tid < E) {
    start[tid] = excl;
    counts[tid] = total;
    offsets[tid] = excl;
  }
  if (tid == kPermSingle - 1) offsets[E] = before + incl;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r * kPermSingle + tid >= V) continue;
    const int64_t ts = static_cast<int64_t>(t[r]) * k + s[r];
    if (!valid[r]) {
      inv[ts] = -1;
    } else {
      const int pos = start[e[r]] + cnt[r * kW + wave][e[r]] + rank[r];
      perm_tok[pos] = t[r];
      perm_slot[pos] = s[r];
      inv[ts] = pos;
    }
  }
}

template <int IB, int R, int EMAX>
__global__ __launch_bounds__(kPermSingle) void perm_single(const void* idx, int T, int k, int E,
                                                           int nbits, int V, int32_t* counts,
                                                           int32_t* offsets, int32_t* perm_tok,
                                                           int32_t* perm_slot, int32_t* inv) {
  perm_single_body<IB, R, EMAX>(idx, T, k, E, nbits, V, counts, offsets, perm_tok, perm_slot, inv);
}

// Route and permutation of a small batch (route_perm_small_supported) in one workgroup: wave t selects token t's experts (route_token), the indices go
// to LDS and to idx, and after a barrier the workgroup permutes them as perm_single does.
// Saves a launch on the decode path of small batches.
template <int EPL>
__global__ __launch_bounds__(kPermSingle) void route_perm_small(
    const uint16_t* __restrict__ logits, const float* __restrict__ bias,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w_sg, int T, int E, int H, int k,
    int nbits, int32_t* __restrict__ idx, uint16_t* __restrict__ topw, float* __restrict__ sgate,
    int32_t* counts, int32_t* offsets, int32_t* perm_tok, int32_t* perm_slot, int32_t* inv) {
  __shared__ int32_t s_idx[kPermSingle];
  const int wave = threadIdx.x / kWave;
  if (wave < T)                                             // the same for the whole wave
    route_token<EPL>(logits, bias, x, w_sg, wave, E, H, k, s_idx, 4, topw, sgate);
  __syncthreads();
  const int V = T * k;
  if (static_cast<int>(threadIdx.x) < V) idx[threadIdx.x] = s_idx[threadIdx.x];
  perm_single_body<4, 1, 1024>(s_idx, T, k, E, nbits, V, counts, offsets, perm_tok, perm_slot,
                               inv);
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* p, int64_t n, int32_t value) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = value;
}

hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  fill_i32_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(p, n, value);
  return hipGetLastError();
}

static int bits_for(int E) {
  int n = 0;
  while ((1 << n) < E) ++n;
  return n;
}

template <int IB>
static hipError_t launch_permute_t(const void* idx, int64_t T, int k, int E, int32_t* counts,
                                   int32_t* offsets, int32_t* perm_tok, int32_t* perm_slot,
                                   int32_t* inv, int32_t* hist, int32_t* base, int32_t* lrank,
                                   hipStream_t s) {
  const int V = static_cast<int>(T * k);
  const int nbits = bits_for(E);
  // one workgroup up to 2 (4 for E <= 512) entries per thread; the LDS count table is
  // (16 * R) x EMAX ints, at most 128 KB
  auto single = [&]<int R, int EMAX>() {
    perm_single<IB, R, EMAX><<<1, kPermSingle, 0, s>>>(idx, static_cast<int>(T), k, E, nbits, V,
                                                       counts, offsets, perm_tok, perm_slot, inv);
    return hipGetLastError();
  };
  if (V <= kPermSingle) return single.template operator()<1, 1024>();
  if (V <= 2 * kPermSingle) return single.template operator()<2, 1024>();
  if (V <= 4 * kPermSingle && E <= 512) return single.template operator()<4, 512>();
  // hist, base: E x nblk; lrank: V; the per-expert totals are the counts
  const int nblk = static_cast<int>(perm_blocks(V));
  perm_count<IB><<<nblk, 64, 0, s>>>(idx, static_cast<int>(T), k, E, nbits, V, nblk, hist,
                                     lrank);
  launch_expert_scan(hist, nblk, E, base, counts, s);
  perm_scatter<IB><<<nblk, 64, 0, s>>>(idx, static_cast<int>(T), k, E, V, nblk, base, counts,
                                       offsets, lrank, perm_tok, perm_slot, inv);
  return hipGetLastError();
}

bool perm_chunked(int64_t V, int E) {
  return V > 2 * kPermSingle && !(V <= 4 * kPermSingle && E <= 512);
}

hipError_t launch_perm_count_scan(const void* idx, int idx_bytes, int64_t T, int k, int E,
                                  int32_t* hist, int32_t* base, int32_t* lrank, int32_t* counts,
                                  hipStream_t s) {
  const int V = static_cast<int>(T * k), nbits = bits_for(E);
  const int nblk = static_cast<int>(perm_blocks(V));
  if (idx_bytes == 8)
    perm_count<8><<<nblk, 64, 0, s>>>(idx, static_cast<int>(T), k, E, nbits, V, nblk, hist, lrank);
  else
    perm_count<4><<<nblk, 64, 0, s>>>(idx, static_cast<int>(T), k, E, nbits, V, nblk, hist, lrank);
  launch_expert_scan(hist, nblk, E, base, counts, s);
  return hipGetLastError();
}

hipError_t launch_perm_scan(const int32_t* hist, int nchunks, int E, int32_t* base,
                            int32_t* totals, hipStream_t s) {
  launch_expert_scan(hist, nchunks, E, base, totals, s);
  return hipGetLastError();
}

hipError_t launch_permute(const void* idx, int idx_bytes, int64_t T, int k, int E,
                          bool /*shared_rows*/, int32_t* counts, int32_t* offsets,
                          int32_t* perm_tok, int32_t* perm_slot, int32_t* inv, int32_t* hist,
                          int32_t* base, int32_t* lrank, hipStream_t s) {
  if (idx_bytes == 8)
    return launch_permute_t<8>(idx, T, k, E, counts, offsets, perm_tok, perm_slot, inv, hist,
                               base, lrank, s);
  return launch_permute_t<4>(idx, T, k, E, counts, offsets, perm_tok, perm_slot, inv, hist,
                             base, lrank, s);
}

// The fused kernel runs every token's selection on one CU: past 4 tokens that only pays while
// each selection is short (E <= 128; at E = 512, T = 16 it was 2 us slower than two kernels).
bool route_perm_small_supported(int64_t T, int k, int E) {
  return T >= 1 && T <= (E <= 128 ? kSmallRouteTokens : 4) && T * k <= kPermSingle && E <= 1024;
}

hipError_t launch_route_perm_small(const void* logits, const float* bias, const void* x,
                                   const void* w_sg, int64_t T, int E, int H, int k, int32_t* idx,
                                   void* topw, float* sgate, int32_t* counts, int32_t* offsets,
                                   int32_t* perm_tok, int32_t* perm_slot, int32_t* inv,
                                   hipStream_t s) {
  const auto* lg = static_cast<const uint16_t*>(logits);
  const auto* xx = static_cast<const uint16_t*>(x);
  const auto* ws = static_cast<const uint16_t*>(w_sg);
  auto* tw = static_cast<uint16_t*>(topw);
  const int Ti = static_cast<int>(T), nbits = bits_for(E);
#define LBMOE_ROUTE_PERM(EPL)                                                                  \
  route_perm_small<EPL><<<1, kPermSingle, 0, s>>>(lg, bias, xx, ws, Ti, E, H, k, nbits, idx, tw, \
                                                  sgate, counts, offsets, perm_tok, perm_slot, inv)
  if (E <= 64) LBMOE_ROUTE_PERM(1);
  else if (E <= 128) LBMOE_ROUTE_PERM(2);
  else if (E <= 256) LBMOE_ROUTE_PERM(4);
  else if (E <= 512) LBMOE_ROUTE_PERM(8);
  else LBMOE_ROUTE_PERM(16);
#undef LBMOE_ROUTE_PERM
  return hipGetLastError();
}

}  // namespace lbmoe
