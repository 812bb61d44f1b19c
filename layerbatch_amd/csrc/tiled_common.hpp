// Helpers shared by the LDS-tiled kernels (tiled_gemm.hip, tiled_fp8.hip).
#pragma once

#include "common.hpp"

namespace lbmoe {

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Workgroup barrier for the LDS ring: the wave's LDS reads are complete (lgkmcnt 0) and its
// own global->LDS copies were waited for by the caller; unlike __syncthreads this does not
// drain the copies still in flight for later stages. The signal fences keep the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((0x3f & 0xf) | ((0x3f >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until the oldest in-flight stage's copies (L copies per stage and wave) have landed
// while the copies of up to min(S, later) younger stages stay in flight (vector-memory
// operations complete in order).
template <int S, int L>
__device__ __forceinline__ void wait_ring(int later) {
  static_assert(S * L < 64, "vmcnt holds at most 63 outstanding operations");
  if constexpr (S <= 0) {
    wait_vmcnt<0>();
  } else {
    if (later >= S) wait_vmcnt<S * L>();
    else wait_ring<S - 1, L>(later);
  }
}

// Buffer resource for raw accesses (stride 0, no swizzle) at byte offsets below 2^31 from
// `base`, which must be wave-uniform; readfirstlane makes that visible to the compiler, so the
// descriptor lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo), 0, 0x7fffffff, 0x00020000);
}

// Workgroup b runs on XCD b % 8. The first `items` work items are spread over the 8 XCDs in
// contiguous chunks, so consecutive items (which share operands) run together on one XCD's L2
// and every XCD gets an equal share however much larger than `items` the grid is. Returns the
// item of workgroup b, or -1 when b has none. The grid must hold at least round8(items)
// workgroups.
__device__ __forceinline__ int xcd_item(int b, int items) {
  const int chunk = (items + 7) >> 3;
  const int j = b >> 3;
  if (j >= chunk) return -1;
  const int item = (b & 7) * chunk + j;
  return item < items ? item : -1;
}

inline unsigned round8(int64_t v) { return static_cast<unsigned>((v + 7) / 8 * 8); }

}  // namespace lbmoe
