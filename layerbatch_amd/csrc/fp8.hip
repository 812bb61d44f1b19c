// fp8 (OCP e4m3fn) quantisation kernels. The reference has no fp8 path; these define the
// quantised variant: weights per 128x128 block and activations per (row, 128 channels), with
// scale = amax / 448 (an all-zero block gets scale 1) and code = e4m3(value / scale) rounded
// to nearest even and saturated to +-448.
#include "common.hpp"
#include "internal.hpp"

namespace lbmoe {

__device__ __forceinline__ float scale_of(float amax) { return amax > 0.f ? amax / 448.0f : 1.0f; }

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
  const float s = scale_of(amax);
  if (threadIdx.x == 0) scale[blk] = s;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t lo = v[i + h][2 * j], hi = v[i + h][2 * j + 1];
        o[2 * h + j] = f2e4m3(bf_lo(lo) / s) | (f2e4m3(bf_hi(lo) / s) << 8) |
                       (f2e4m3(bf_lo(hi) / s) << 16) | (f2e4m3(bf_hi(hi) / s) << 24);
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

// One wave per (row, 128-channel group); lane i covers channels 2i, 2i+1.
__global__ __launch_bounds__(256) void quant_groups_kernel(const uint16_t* __restrict__ a,
                                                           int64_t rows, int cols, int ld,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale) {
  const int ng = cols / 128;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (gid >= rows * ng) return;
  const int64_t row = gid / ng;
  const int grp = static_cast<int>(gid - row * ng);
  const int lane = lane_id();
  const uint32_t v = *reinterpret_cast<const uint32_t*>(a + row * ld + grp * 128 + 2 * lane);
  const float x0 = bf_lo(v), x1 = bf_hi(v);
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const float s = scale_of(amax);
  if (lane == 0) scale[row * ng + grp] = s;
  const uint32_t c = f2e4m3(x0 / s) | (f2e4m3(x1 / s) << 8);
  *reinterpret_cast<uint16_t*>(q + row * cols + grp * 128 + 2 * lane) = static_cast<uint16_t>(c);
}

hipError_t launch_quant_groups_fp8(const void* a, int64_t rows, int cols, int ld, void* q,
                                   float* scale, hipStream_t s) {
  const int64_t waves = rows * (cols / 128);
  if (waves == 0) return hipSuccess;
  quant_groups_kernel<<<static_cast<unsigned>((waves + 3) / 4), 256, 0, s>>>(
      static_cast<const uint16_t*>(a), rows, cols, ld, static_cast<uint8_t*>(q), scale);
  return hipGetLastError();
}

}  // namespace lbmoe
