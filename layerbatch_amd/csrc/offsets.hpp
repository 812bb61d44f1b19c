// Host-side limits of the LDS-tiled GEMMs' operand addressing (tiled_gemm.hip, tiled_fp8.hip).
//
// Their global->LDS copies go through raw buffer resources whose range is 0x7fffffff bytes
// (raw_rsrc): a lane's 32-bit byte offset plus the k-tile step carried in the scalar offset
// must stay below 2^31, or the hardware returns zeros for the copy. Every copy reads inside
// one operand matrix (a weight matrix, the token rows x / xq, or the act rows act / actq), so
// bounding each matrix's whole byte extent bounds every offset the copies form, the k-tile
// steps included. Batches past these limits take the weight-streaming GEMMs, which address
// with 64-bit pointers.
//
// Plain C++ with no HIP dependency, so the limits can be checked by a host compiler alone.
#pragma once

#include <stdint.h>

namespace lbmoe {

constexpr int64_t kTiledMaxBytes = int64_t{1} << 31;

// bf16 operands: x [T, H], act [T*(k+1), Imax] (routed rows plus the shared expert's T rows),
// and one expert's gate_up [2*I, H] (the gate and the up half are separate bases of I*H) or
// down [H, I] matrix.
inline bool bf16_tiled_offsets_fit(int64_t T, int64_t k, int64_t H, int64_t Imax) {
  return T * H * 2 < kTiledMaxBytes && T * (k + 1) * Imax * 2 < kTiledMaxBytes &&
         Imax * H * 2 < kTiledMaxBytes;
}

// e4m3 operands: xq [T, H], actq [rows, Imax], one expert's gate_up [2*I, H] bytes; the scale
// rows are four bytes per 128 values and so lie far inside the same bound.
inline bool fp8_tiled_offsets_fit(int64_t T, int64_t rows, int64_t H, int64_t Imax) {
  return T * H < kTiledMaxBytes && rows * Imax < kTiledMaxBytes &&
         2 * Imax * H < kTiledMaxBytes;
}

}  // namespace lbmoe
