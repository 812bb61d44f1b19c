// One token's router selection, executed by one wave: softmax -> top-k -> renormalise -> bf16
// and the shared-expert gate (the algorithm and its reference lines are described in
// route.hip). Shared by the route kernel, the fused route + permutation kernel of small
// batches, the decode gate_up kernel that routes inline, and the tiled router that selects
// from its own logits.
#pragma once

#include <float.h>

#include "common.hpp"

namespace lbmoe {

// Order-preserving map float -> uint32 (larger float -> larger key); -0 maps with +0.
__device__ __forceinline__ uint32_t order_key(float z) {
  const uint32_t u = __float_as_uint(z + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// v of another lane of the row (DPP control CTRL), every lane of the row taking part.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// Wave-wide maximum of v (DPP within each 16-lane row, then the four row maxima).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xf, 0xf, false)));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}
__device__ __forceinline__ int wave_min_i32(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xf, 0xf, false));
  const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return min(min(r0, r1), min(r2, r3));
}

// Packed keys for scores that are bf16 values (routers without a bias): the order key of a
// bf16 value has 16 low bits that are the same for every value of its sign, so they can carry
// 1023 - e instead. Every expert's key is then distinct, a larger key is exactly an earlier
// place in the (descending score, ascending expert) order, the expert comes back from the low
// bits, and the score's bf16 bits from the high ones (packed_score). 0 is below every key.
__device__ __forceinline__ uint32_t packed_key(float z, int e) {
  return (order_key(z) & 0xffff0000u) | static_cast<uint32_t>(1023 - e);
}
__device__ __forceinline__ float packed_score(uint32_t key) {
  const uint32_t u = (key & 0x80000000u) ? (key & 0x7fff0000u) : (~key & 0xffff0000u);
  return __uint_as_float(u);
}
__device__ __forceinline__ int packed_expert(uint32_t key) {
  return 1023 - static_cast<int>(key & 1023u);
}

// Sorts n keys descending with Batcher's odd-even merge network (n a power of two, all
// indices compile-time, so the keys stay in registers: 19 compare-exchanges for 8 keys).
template <int N>
__device__ __forceinline__ void sort_desc(uint32_t (&key)[N]) {
  static_assert((N & (N - 1)) == 0, "a power of two");
#pragma unroll
  for (int p = 1; p < N; p <<= 1)
#pragma unroll
    for (int kk = p; kk >= 1; kk >>= 1)
#pragma unroll
      for (int j = kk % p; j + kk < N; j += 2 * kk)
#pragma unroll
        for (int i = 0; i < kk; ++i) {
          const int a = i + j, b = i + j + kk;
          if (b < N && a / (2 * p) == b / (2 * p)) {
            const uint32_t hi = max(key[a], key[b]), lo = min(key[a], key[b]);
            key[a] = hi;
            key[b] = lo;
          }
        }
}

// Removes the first of a lane's keys when it is the round's winner: with keep = 0 on that lane
// and all ones elsewhere, each key becomes a bitfield blend of itself and its successor (one
// v_bfi_b32). (A select between neighbouring elements is turned by the compiler into an indexed
// read of the array, a chain of compares per element.)
template <int N>
__device__ __forceinline__ void pop_if(uint32_t (&key)[N], uint32_t winner) {
  const uint32_t keep = key[0] == winner ? 0u : 0xffffffffu;
#pragma unroll
  for (int j = 0; j + 1 < N; ++j) key[j] = (key[j] & keep) | (key[j + 1] & ~keep);
  key[N - 1] &= keep;
}

// Wave-wide maximum of v, uniform: DPP within each 16-lane row, then the row broadcasts 15 and
// 31 carry the maximum into lane 63.
// Rows a broadcast leaves out read 0, which the maximum ignores.
__device__ __forceinline__ uint32_t wave_max_u32_bcast(uint32_t v) {
  v = max(v, static_cast<uint32_t>(dpp_i32<0xb1>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i32<0x4e>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i32<0x141>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i32<0x140>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false)));
  return __builtin_amdgcn_readlane(v, 63);
}

// Selection from one token's scores, z[j] = logit + bias of expert j * 64 + lane (-inf past E
// and for NaN), every lane of the wave calling it: writes idx_out[o + s] (idx_bytes 4 or 8),
// topw[o + s] (when not null) and idx_lds[s] (a second copy of the ids, when not null), o = t*k.
// bf16_scores (wave-uniform): every z is a bf16 value (no bias was added), which allows the
// packed keys: each lane sorts its keys once, and a round is a wave maximum of the lanes' first
// keys, after which the winning lane drops its first key.
template <int EPL>
__device__ __forceinline__ void route_select(const float (&z)[EPL], int E, int k, int64_t o,
                                             void* idx_out, int idx_bytes,
                                             uint16_t* __restrict__ topw, int32_t* idx_lds,
                                             bool bf16_scores = false) {
  const int lane = lane_id();
  uint32_t key[EPL];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    key[j] = e < E ? (bf16_scores ? packed_key(z[j], e) : order_key(z[j])) : 0u;
    m = fmaxf(m, z[j]);
  }
  m = wave_max_dpp(m);
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    if (j * kWave + lane < E) part += expf(z[j] - m);
  const float S = wave_sum_dpp(part);

  // k rounds of argmax; lane r < k keeps round r's winner (expert and key)
  int my_e = 0;
  uint32_t my_key = 0;
  if (bf16_scores) {
    sort_desc<EPL>(key);
    for (int r = 0; r < k; ++r) {
      const uint32_t wmax = wave_max_u32_bcast(key[0]);
      pop_if<EPL>(key, wmax);
      if (lane == r) my_key = wmax;
    }
    my_e = packed_expert(my_key);
  }
  for (int r = 0; r < (bf16_scores ? 0 : k); ++r) {
    uint32_t best = key[0];
    int bj = 0;
#pragma unroll
    for (int j = 1; j < EPL; ++j)
      if (key[j] > best) {
        best = key[j];
        bj = j;
      }
    const uint32_t wmax = wave_max_u32(best);
    const uint64_t holders = __ballot(best == wmax);
    int win;                                            // winning expert
    if (__popcll(holders) == 1) {
      const int wl = __builtin_ctzll(holders);
      win = __builtin_amdgcn_readlane(bj * kWave + lane, wl);
    } else {
      win = wave_min_i32(best == wmax ? bj * kWave + lane : 0x7fffffff);
    }
    const int wj = win / kWave, wl = win % kWave;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (j == wj && lane == wl) key[j] = 0u;
    if (lane == r) {
      my_e = win;
      my_key = wmax;
    }
  }
  float p = 0.f;
  if (lane < k) {
    const uint32_t u = (my_key & 0x80000000u) ? (my_key & 0x7fffffffu) : ~my_key;   // key -> z
    p = expf((bf16_scores ? packed_score(my_key) : __uint_as_float(u)) - m) / S;
  }
  const float psum = wave_sum_dpp(p);
  if (lane < k) {
    if (topw != nullptr) topw[o + lane] = static_cast<uint16_t>(f2bf(p / psum));
    if (idx_bytes == 8) reinterpret_cast<int64_t*>(idx_out)[o + lane] = my_e;
    else reinterpret_cast<int32_t*>(idx_out)[o + lane] = my_e;
    if (idx_lds != nullptr) idx_lds[lane] = my_e;
  }
}

// Reductions over the 8-lane groups of a wave (lanes 8g .. 8g+7): two quad swaps, then the
// mirror within each half row, after which every lane of the group holds the result.
__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, dpp_f32<0xb1>(v));
  v = fmaxf(v, dpp_f32<0x4e>(v));
  return fmaxf(v, dpp_f32<0x141>(v));
}
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp_f32<0xb1>(v);
  v += dpp_f32<0x4e>(v);
  return v + dpp_f32<0x141>(v);
}
__device__ __forceinline__ uint32_t group8_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(dpp_i32<0xb1>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i32<0x4e>(static_cast<int>(v))));
  return max(v, static_cast<uint32_t>(dpp_i32<0x141>(static_cast<int>(v))));
}
__device__ __forceinline__ int group8_min_i32(int v) {
  v = min(v, dpp_i32<0xb1>(v));
  v = min(v, dpp_i32<0x4e>(v));
  return min(v, dpp_i32<0x141>(v));
}

// route_select for 8 tokens at once, one per 8-lane group: lane u of a group holds the scores
// of experts u, u + 8, ..., z[j] of expert 8j + u (-inf past E and for NaN), and the group's
// reductions stay within it, so a wave selects 8 tokens in the time route_select takes for
// one. The same order (descending score, ties to the lower expert); the softmax sums run in
// another order, so a weight may differ from route_select's by one bf16 step. Lane u writes
// slots u and u + 8 (k <= 16): idx_out[o + s], topw[o + s] (when not null) and idx_lds[s]
// (when not null); lanes with write == false only take part in the reductions.
// bf16_scores: as for route_select, packed keys sorted once per lane.
template <int EPG>
__device__ __forceinline__ void route_select8(const float (&z)[EPG], int E, int k, int64_t o,
                                              bool write, int32_t* __restrict__ idx_out,
                                              uint16_t* __restrict__ topw, int32_t* idx_lds,
                                              bool bf16_scores = false) {
  const int u = lane_id() & 7;
  uint32_t key[EPG];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPG; ++j) {
    const int e = 8 * j + u;
    key[j] = e < E ? (bf16_scores ? packed_key(z[j], e) : order_key(z[j])) : 0u;
    m = fmaxf(m, z[j]);
  }
  m = group8_max(m);
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < EPG; ++j)
    if (8 * j + u < E) part += expf(z[j] - m);
  const float S = group8_sum(part);
  int my_e[2] = {0, 0};
  uint32_t my_key[2] = {0u, 0u};
  if (bf16_scores) {
    sort_desc<EPG>(key);
    for (int r = 0; r < k; ++r) {
      const uint32_t gmax = group8_max_u32(key[0]);
      pop_if<EPG>(key, gmax);
      if ((r & 7) == u) {
        my_e[r >> 3] = packed_expert(gmax);
        my_key[r >> 3] = gmax;
      }
    }
  }
  for (int r = 0; r < (bf16_scores ? 0 : k); ++r) {
    uint32_t best = key[0];
    int bj = 0;
#pragma unroll
    for (int j = 1; j < EPG; ++j)
      if (key[j] > best) {
        best = key[j];
        bj = j;
      }
    const uint32_t gmax = group8_max_u32(best);
    const int win = group8_min_i32(best == gmax ? 8 * bj + u : 0x7fffffff);
#pragma unroll
    for (int j = 0; j < EPG; ++j)
      if (8 * j + u == win) key[j] = 0u;
    if ((r & 7) == u) {
      my_e[r >> 3] = win;
      my_key[r >> 3] = gmax;
    }
  }
  float p[2], ps = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t kk = my_key[h];
    const uint32_t bits = (kk & 0x80000000u) ? (kk & 0x7fffffffu) : ~kk;   // key -> z
    const float zk = bf16_scores ? packed_score(kk) : __uint_as_float(bits);
    p[h] = u + 8 * h < k ? expf(zk - m) / S : 0.f;
    ps += p[h];
  }
  const float psum = group8_sum(ps);
  if (!write) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = u + 8 * h;
    if (r < k) {
      if (topw != nullptr) topw[o + r] = static_cast<uint16_t>(f2bf(p[h] / psum));
      idx_out[o + r] = my_e[h];
      if (idx_lds != nullptr) idx_lds[r] = my_e[h];
    }
  }
}

// sgate[t] = sigmoid(bf16(x[t] . w_sg)), every lane of the wave calling it. With xq (fp8
// layers): the row's e4m3 codes and per-128-channel scales as well, as quant_groups_kernel
// writes them (xq[t, :], xs[t, H / 128]). A load of the loop covers channels 8 lane + 512 i, so
// the 16 lanes of a DPP row hold exactly one 128-channel group: the row is quantised from the
// registers the dot product reads, and its separate pass over x is saved.
__device__ __forceinline__ void shared_gate(const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ w_sg, int t, int H,
                                            float* __restrict__ sgate,
                                            uint8_t* __restrict__ xq = nullptr,
                                            float* __restrict__ xs = nullptr) {
  const int lane = lane_id();
  const uint16_t* xr = x + static_cast<int64_t>(t) * H;
  float d = 0.f;
  for (int c = lane * 8; c < H; c += kWave * 8) {
    const u32x4 a = ld16(xr + c);
    const u32x4 b = ld16(w_sg + c);
    if (xq != nullptr) {                 // whole DPP rows are active: H is a multiple of 128
      float sc;
      const u32x2 q = quant_group16(a, sc);
      *reinterpret_cast<u32x2*>(xq + static_cast<int64_t>(t) * H + c) = q;
      if ((lane & 15) == 0) xs[static_cast<int64_t>(t) * (H / 128) + c / 128] = sc;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      d += bf_lo(a[q]) * bf_lo(b[q]);
      d += bf_hi(a[q]) * bf_hi(b[q]);
    }
  }
  d = round_bf(wave_sum_dpp(d));
  if (lane == 0) sgate[t] = 1.0f / (1.0f + expf(-d));
}

// Token t's selection: idx_out[t*k + s] (idx_bytes 4 or 8), topw[t*k + s] and sgate[t] (each
// when not null). Every lane of the wave must call it; it uses no LDS and no barrier.
template <int EPL>
__device__ __forceinline__ void route_token(const uint16_t* __restrict__ logits,
                                            const float* __restrict__ bias,
                                            const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ w_sg, int t, int E,
                                            int H, int k, void* idx_out, int idx_bytes,
                                            uint16_t* __restrict__ topw,
                                            float* __restrict__ sgate,
                                            uint8_t* __restrict__ xq = nullptr,
                                            float* __restrict__ xs = nullptr) {
  const int lane = lane_id();
  const uint16_t* lrow = logits + static_cast<int64_t>(t) * E;
  // unconditional loads (lanes past E read expert E-1 and are masked): a load under a
  // condition would make the compiler wait for it before the next one is issued
  uint16_t lv[EPL];
  float bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = min(j * kWave + lane, E - 1);
    lv[j] = lrow[e];
    bv[j] = bias ? bias[e] : 0.f;
  }
  float z[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = j * kWave + lane;
    const float v = bf2f(lv[j]) + bv[j];
    z[j] = (!(v == v) || e >= E) ? -INFINITY : v;      // a NaN logit is never preferred
  }
  // the shared-expert gate, its loads in flight together with the logits'
  if (sgate != nullptr) shared_gate(x, w_sg, t, H, sgate, xq, xs);
  route_select<EPL>(z, E, k, static_cast<int64_t>(t) * k, idx_out, idx_bytes, topw, nullptr,
                    bias == nullptr);
}

}  // namespace lbmoe
