// Pre-pass of the packed parallel kernel (d = 16, bf16).  Per 64-key block of a head it writes
//  * V (bf16 [N][dv]) as an fp16 V^T block [DV rows][ROW halves], rounded up to whole 1 KB units
//    so that the main kernel copies a block straight into LDS with buffer_load ... lds;
//  * the block's statistics, a record of stats_width(DV) floats: the column sums of V (DV), the
//    sums of k (16) and the upper triangle of sum k k^T (136 entries, row-major, off-diagonal
//    entries doubled), then zero padding.  A scan turns the records into exclusive prefixes over
//    the blocks, from which the main kernel takes everything a query needs of the blocks before
//    its diagonal block except the P.V products themselves.
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

constexpr int kStatK1 = 0;     // offset of the k sums after the V column sums
constexpr int kStatK2 = 16;    // offset of the k k^T triangle after the V column sums
constexpr int kTri = 136;      // entries of the triangle (16 * 17 / 2)
__host__ __device__ constexpr int stats_width(int DV) { return DV + 160; }

// One work-group per (64-key block, head); k rows are d = 16 bf16 (8-byte aligned).  Zero for
// keys >= N, rows >= dv and the padding.  VEC: dv even and v 4-byte aligned (pairs of V are
// loaded as one dword).
template <int DV, int ROW, bool VEC>
__global__ __launch_bounds__(256) void par_pack_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                       uint16_t* __restrict__ vt, float* __restrict__ stats, int N,
                                                       int dv, int nb64) {
  constexpr int NP = 256 / DV;   // partial sums per column
  constexpr int SW = stats_width(DV);
  __shared__ float tile[BN][DV + 1];
  __shared__ float ktile[BN][17];
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
  // k: thread -> key tid / 4, dims 4 (tid % 4) .. +3
  u32x2 kx = {0u, 0u};
  {
    const int key = tid >> 2;
    if (row0 + key < N)
      kx = *reinterpret_cast<const u32x2*>(k + ((size_t)bh * N + row0 + key) * 16 + 4 * (tid & 3));
  }
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int idx = tid + 256 * i, key = idx / (DV / 2), col = 2 * (idx % (DV / 2));
    tile[key][col] = bf16_lo_to_f32(x[i]);
    tile[key][col + 1] = bf16_hi_to_f32(x[i]);
  }
  {
    float* kr = &ktile[tid >> 2][4 * (tid & 3)];
    kr[0] = bf16_lo_to_f32(kx[0]);
    kr[1] = bf16_hi_to_f32(kx[0]);
    kr[2] = bf16_lo_to_f32(kx[1]);
    kr[3] = bf16_hi_to_f32(kx[1]);
  }
  __syncthreads();
  u32* __restrict__ dst = reinterpret_cast<u32*>(vt + ((size_t)bh * nb64 + blk) * (VtBlock<DV, ROW>::bytes / 2));
  for (int idx = tid; idx < VtBlock<DV, ROW>::bytes / 4; idx += 256) {
    const int row = (2 * idx) / ROW, col = (2 * idx) % ROW;
    u32 y = 0u;
    if (row < DV && col < BN) y = pack_f16x2(tile[col][row], tile[col + 1][row]);
    dst[idx] = y;
  }
  float* __restrict__ rec = stats + ((size_t)bh * nb64 + blk) * SW;
  {
    const int col = tid % DV, pi = tid / DV;
    float t = 0.f;
#pragma unroll
    for (int key = pi * (BN / NP); key < (pi + 1) * (BN / NP); ++key) t += tile[key][col];
    part[pi][col] = t;
  }
  if (tid < kTri) {
    // triangle entry tid -> (a, b), a <= b, row-major
    int a = 0, t = tid;
    while (t >= 16 - a) {
      t -= 16 - a;
      ++a;
    }
    const int b = a + t;
    float s = 0.f;
#pragma unroll 16
    for (int key = 0; key < BN; ++key) s = __builtin_fmaf(ktile[key][a], ktile[key][b], s);
    rec[DV + kStatK2 + tid] = a == b ? s : 2.f * s;
  } else if (tid < kTri + 16) {
    const int a = tid - kTri;
    float s = 0.f;
#pragma unroll 16
    for (int key = 0; key < BN; ++key) s += ktile[key][a];
    rec[DV + kStatK1 + a] = s;
  } else if (tid < kTri + 24) {
    rec[DV + kStatK2 + kTri + (tid - kTri - 16)] = 0.f;
  }
  __syncthreads();
  if (tid < DV) {
    float t = 0.f;
#pragma unroll
    for (int pi = 0; pi < NP; ++pi) t += part[pi][tid];
    rec[tid] = t;
  }
}

// stats[bh][blk][sw] -> exclusive prefix over blk, in place.  Work-group (bh, g) scans columns
// 16 g .. 16 g + 15 of head bh in tiles of 256 blocks: 16 threads per column each sum a run of 16
// blocks, a 16-term scan of the run totals gives each run's offset, and a carry links the tiles.
__global__ __launch_bounds__(256) void stats_scan_kernel(float* __restrict__ stats, int nb64, int sw) {
  constexpr int CW = 16, NT = 256 / CW, TB = 256, PER = TB / NT;
  __shared__ float tile[TB][CW + 1];
  __shared__ float tot[NT][CW];
  const int tid = threadIdx.x, col = tid % CW, g = tid / CW;
  float* __restrict__ s = stats + (size_t)blockIdx.x * nb64 * sw + CW * blockIdx.y;
  float carry = 0.f;
  for (int t0 = 0; t0 < nb64; t0 += TB) {
    const int nt = min(TB, nb64 - t0);
    float x[TB * CW / 256];
#pragma unroll
    for (int i = 0; i < TB * CW / 256; ++i) {   // all loads in flight before the first LDS store
      const int bl = g + NT * i;
      x[i] = bl < nt ? s[(size_t)(t0 + bl) * sw + col] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < TB * CW / 256; ++i) tile[g + NT * i][col] = x[i];
    __syncthreads();
    float run = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) run += tile[g * PER + i][col];
    tot[g][col] = run;
    __syncthreads();
    run = carry;
    float all = carry;
#pragma unroll
    for (int g2 = 0; g2 < NT; ++g2) {
      const float t = tot[g2][col];
      if (g2 < g) run += t;
      all += t;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float t = tile[g * PER + i][col];
      tile[g * PER + i][col] = run;
      run += t;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TB * CW / 256; ++i) {
      const int bl = g + NT * i;
      if (bl < nt) s[(size_t)(t0 + bl) * sw + col] = tile[bl][col];
    }
    carry = all;
    __syncthreads();
  }
}

}  // namespace
}  // namespace la
