// The 48 x 64 F32-MFMA output tile of the narrow linear (linear_api.hip);
// the pipelined patch embedding (patch_embed.hip) keeps its wave layout and
// fragment order.
//
// Eight MFMA waves (two per SIMD) compute a 48 x 64 tile: wave w computes the
// 48 x 16 strip w%4 (three 16x16 accumulators) over one half of K (split-K
// inside the workgroup); the two partial sums meet in LDS before the
// epilogue.  Two waves per SIMD let one wave's MFMAs run while the other
// waits on memory.
//
// Fragment order.  v_mfma_f32_16x16x4_f32 takes, in lane l, A[l%16][k] and
// B[k][l%16] for the lane's k = one of 4 per step (lane group g = l/16).  K is
// walked in blocks of 16: in block b, lane group g holds k = 16b + 4g + j in
// component j of a 128-bit read, and step j of the block multiplies component
// j, so four steps cover the block's 16 k once and one ds_read_b128 feeds
// four MFMAs.  With LDS rows k-contiguous and a row pitch of 4 x odd floats,
// the 16 rows of a fragment read start on 16 distinct 4-bank groups: no bank
// conflicts.
#pragma once

#include "common.h"

namespace vkm {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 48;
constexpr int BN = 64;
constexpr int kThreads = 512;
constexpr int kKAlign = 16;  // weight rows are zero-padded to a 16-block

__device__ __forceinline__ void mfma_block(const float* arow, int t_pitch, const f32x4& b,
                                           f32x4 acc[3]) {
  f32x4 a[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) a[t] = *reinterpret_cast<const f32x4*>(arow + t * t_pitch);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int t = 0; t < 3; ++t)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][j], b[j], acc[t], 0, 0, 0);
}

// Split-K reduction: waves 4-7 hand their partial sums to waves 0-3.  Returns
// false in waves 4-7, which are then done.
__device__ __forceinline__ bool reduce_halves(float* red, int strip, int half, int lane,
                                              f32x4 acc[3]) {
  if (half == 1) {
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(strip * 12 + t * 4 + r) * 64 + lane] = acc[t][r];
  }
  __syncthreads();
  if (half == 1) return false;
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] += red[(strip * 12 + t * 4 + r) * 64 + lane];
  return true;
}

}  // namespace vkm
