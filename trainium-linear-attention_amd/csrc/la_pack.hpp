// Pre-pass shared by the packed parallel kernel and the chunked kernels: V (bf16 [N][dv] per
// head) -> fp16 V^T blocks of 64 keys, [DV rows][ROW halves] per block, rounded up to whole 1 KB
// units so that the main kernels can copy a block straight into LDS with buffer_load ... lds.
#pragma once

#include "la_common.hpp"
#include "la_stage.hpp"

namespace la {
namespace {

template <int DV, int ROW>
struct VtBlock {
  static constexpr int units = (DV * ROW * 2 + 1023) / 1024;
  static constexpr int bytes = units * 1024;
};

// One work-group per (64-key block, head).  Zero for keys >= N, rows >= dv and the padding.
// COLSUM: also writes the column sums of the block, colsum[bh][blk][DV].  VEC: dv even and v
// 4-byte aligned (pairs are loaded as one dword).
template <int DV, int ROW, bool COLSUM, bool VEC>
__global__ __launch_bounds__(256) void vt_pack_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ vt,
                                                      float* __restrict__ colsum, int N, int dv, int nb64) {
  constexpr int NP = 256 / DV;   // partial sums per column
  __shared__ float tile[BN][DV + 1];
  __shared__ float part[NP][DV];
  const int blk = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int row0 = blk * BN;
  const uint16_t* __restrict__ src = v + ((size_t)bh * N + row0) * dv;
  constexpr int NLD = BN * (DV / 2) / 256;   // element pairs per thread
  u32 x[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {   // all loads in flight before the first LDS store
    const int idx = tid + 256 * i, key = idx / (DV / 2), col = 2 * (idx % (DV / 2));
    u32 e = 0u;
    if (row0 + key < N) {
      const uint16_t* s = src + (size_t)key * dv + col;
      if (VEC) {
        if (col < dv) e = *reinterpret_cast<const u32*>(s);
      } else {
        e = (col < dv ? (u32)s[0] : 0u) | (col + 1 < dv ? (u32)s[1] << 16 : 0u);
      }
    }
    x[i] = e;
  }
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int idx = tid + 256 * i, key = idx / (DV / 2), col = 2 * (idx % (DV / 2));
    tile[key][col] = bf16_lo_to_f32(x[i]);
    tile[key][col + 1] = bf16_hi_to_f32(x[i]);
  }
  __syncthreads();
  u32* __restrict__ dst = reinterpret_cast<u32*>(vt + ((size_t)bh * nb64 + blk) * (VtBlock<DV, ROW>::bytes / 2));
  for (int idx = tid; idx < VtBlock<DV, ROW>::bytes / 4; idx += 256) {
    const int row = (2 * idx) / ROW, col = (2 * idx) % ROW;
    u32 y = 0u;
    if (row < DV && col < BN) y = pack_f16x2(tile[col][row], tile[col + 1][row]);
    dst[idx] = y;
  }
  if (COLSUM) {
    {
      const int col = tid % DV, pi = tid / DV;
      float t = 0.f;
#pragma unroll
      for (int key = pi * (BN / NP); key < (pi + 1) * (BN / NP); ++key) t += tile[key][col];
      part[pi][col] = t;
    }
    __syncthreads();
    if (tid < DV) {
      float t = 0.f;
#pragma unroll
      for (int pi = 0; pi < NP; ++pi) t += part[pi][tid];
      colsum[((size_t)bh * nb64 + blk) * DV + tid] = t;
    }
  }
}

}  // namespace
}  // namespace la
