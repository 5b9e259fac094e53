// Pre-pass of the packed parallel kernel (d = 16, bf16).  Per 64-key block of a head it writes
//  * V (bf16 [N][dv]) as an fp16 V^T block [DV rows][ROW halves], rounded up to whole 1 KB units
//    so that the main kernel copies a block straight into LDS with buffer_load ... lds;
//  * the block's statistics, a record of stats_width(DV) floats: the column sums of V (DV), the
//    sums of k (16) and the upper triangle of sum k k^T (136 entries, row-major, off-diagonal
//    entries doubled), then eight words: the block's V exponent, the head's V exponent, zeros.
//    A scan turns the sums into exclusive prefixes over the blocks, from which the main kernel
//    takes everything a query needs of the blocks before its diagonal block except the P.V
//    products themselves.
//
// Range of V.  fp16 holds 2^-14 .. 65504 (normal), bf16 2^-126 .. 3.4e38, so V^T is stored as
// fp16(V * 2^-E) with E a multiple of 8 chosen per head: every block first takes the exponent
// e_b = vexp_step(max |v| of the block), which puts the block's largest |v'| in [1/2, 128); the
// scan then sets the head's E = max_b e_b and multiplies the V^T blocks with e_b < E by
// 2^(e_b - E) in place (exact, or the rounding of a direct conversion when values fall below
// 2^-14).  For V of one order of magnitude every block has the same e_b and nothing is rewritten.
// The main kernel multiplies its P.V accumulators by 2^E.  The column sums of V stay fp32 sums
// of the unscaled bf16 values.
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
constexpr int kStatExpB = kStatK2 + kTri;       // the block's V exponent (float), not prefix-summed
constexpr int kStatExpH = kStatK2 + kTri + 1;   // the head's V exponent, written by the scan
__host__ __device__ constexpr int stats_width(int DV) { return DV + 160; }

// Power-of-two step (a multiple of 8) of a V block or head from the bits of max |v| as an fp32
// value: 8 ceil((e - 6) / 8) for max |v| in [2^e, 2^(e+1)), so max |v| * 2^-step lies in
// [1/2, 128); -128 for an all-zero block (below every other step).
__device__ __forceinline__ int vexp_step(u32 absmax_f32_bits) {
  if (absmax_f32_bits == 0u) return -128;
  const int e = (int)(absmax_f32_bits >> 23) - 127;   // subnormal fp32 (from bf16) -> -127
  return 8 * ((e + 1) >> 3);
}

// One work-group per PPW consecutive 64-key blocks of a head (all their loads issued first); k
// rows are d = 16 bf16 (16-byte aligned), v rows dv % 8 == 0 bf16 (8-byte aligned).  Per block:
//  * V^T: thread t takes keys 2 (t / CPR) and 2 (t / CPR) + 1, columns 8 (t % CPR) .. +7, so it
//    holds both halves of 8 fp16 pairs of the transposed block; it writes them into an LDS
//    image of the block (padding zero), which whole-chunk stores then copy out;
//  * column sums of V from the same registers: lane shuffles, then the waves through LDS;
//  * k sums and the k k^T triangle from one 32x32x16 MFMA chain over the 64 keys (wave 0):
//    A = K^T (rows 16..31 zero), B = K with a column of ones at 16, so C[a][b] = (k k^T)[a][b]
//    and C[a][16] = k1[a].
constexpr int PPW = 1;   // blocks per pack work-group

template <int DV, int ROW>
__global__ __launch_bounds__(256) void par_pack_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                       uint16_t* __restrict__ vt, float* __restrict__ stats, int N,
                                                       int dv, int nb64) {
  constexpr int SW = stats_width(DV);
  constexpr int CPR = DV / 8;                 // 8-element column groups per V row
  constexpr int NT = (BN / 2) * CPR;          // threads holding a (key pair, column group)
  constexpr int NWV = NT / 64;                // waves among them
  constexpr int IMG = VtBlock<DV, ROW>::bytes;
  static_assert(ROW % 2 == 0 && NT <= 256, "pack layout");
  __shared__ __attribute__((aligned(16))) u32 img[IMG / 4];
  __shared__ __attribute__((aligned(16))) uint16_t kl[BN * 16];
  __shared__ float csum[NWV][DV];
  __shared__ u32 vmx[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bh = blockIdx.y, blk0 = blockIdx.x * PPW;
  const int nb = min(PPW, nb64 - blk0);
  const int kp = tid / CPR, cg = tid % CPR, col = 8 * cg;

  for (int i = tid; i < IMG / 16; i += 256) reinterpret_cast<u32x4*>(img)[i] = (u32x4){0u, 0u, 0u, 0u};

  u32x4 va[PPW], vb[PPW], kx[PPW];
#pragma unroll
  for (int b = 0; b < PPW; ++b) {
    const int row0 = (blk0 + b) * BN;
    u32x4 x0 = {0u, 0u, 0u, 0u}, x1 = {0u, 0u, 0u, 0u};
    if (b < nb && tid < NT && col < dv) {
      const uint16_t* src = v + ((size_t)bh * N + row0 + 2 * kp) * dv + col;
      if (row0 + 2 * kp < N) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(src), hi = *reinterpret_cast<const u32x2*>(src + 4);
        x0 = (u32x4){lo[0], lo[1], hi[0], hi[1]};
      }
      if (row0 + 2 * kp + 1 < N) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(src + dv), hi = *reinterpret_cast<const u32x2*>(src + dv + 4);
        x1 = (u32x4){lo[0], lo[1], hi[0], hi[1]};
      }
    }
    va[b] = x0;
    vb[b] = x1;
    u32x4 y = {0u, 0u, 0u, 0u};
    if (b < nb && tid < 128 && row0 + (tid >> 1) < N)
      y = *reinterpret_cast<const u32x4*>(k + ((size_t)bh * N + row0 + (tid >> 1)) * 16 + 8 * (tid & 1));
    kx[b] = y;
  }

#pragma unroll
  for (int b = 0; b < PPW; ++b) {
    if (b >= nb) break;
    const int blk = blk0 + b;
    {
      // max |v| of the block: bf16 magnitudes compare as integers; per wave, then through LDS
      u32 m = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32 x = va[b][i] & 0x7fff7fffu, y = vb[b][i] & 0x7fff7fffu;
        m = max(m, max(max(x & 0xffffu, x >> 16), max(y & 0xffffu, y >> 16)));
      }
      m = wave_max_u32(m);
      if (lane == 0) vmx[w] = m;
    }
    __syncthreads();   // image zeroed / the previous block's readers done / wave maxima written
    // fp16(v 2^-eb) by ldexp on each value: exact, and finite for an all-zero block (eb = -128)
    const int eb = vexp_step(max(max(vmx[0], vmx[1]), max(vmx[2], vmx[3])) << 16);
    float part[8];
    if (tid < NT) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const u32 a0 = va[b][e >> 1], a1 = vb[b][e >> 1];
        const float f0 = (e & 1) ? bf16_hi_to_f32(a0) : bf16_lo_to_f32(a0);
        const float f1 = (e & 1) ? bf16_hi_to_f32(a1) : bf16_lo_to_f32(a1);
        part[e] = f0 + f1;
        img[(col + e) * (ROW / 2) + kp] = pack_f16x2(__builtin_ldexpf(f0, -eb), __builtin_ldexpf(f1, -eb));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[e] = 0.f;
    }
    if (tid < 128) *reinterpret_cast<u32x4*>(&kl[8 * tid]) = kx[b];
    // column sums: lanes with the same column group differ by multiples of CPR
#pragma unroll
    for (int sh = CPR; sh < 64; sh <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) part[e] += __shfl_xor(part[e], sh);
    if (w < NWV && lane < CPR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) csum[w][8 * lane + e] = part[e];
    }
    __syncthreads();
    u32* dst = reinterpret_cast<u32*>(vt + ((size_t)bh * nb64 + blk) * (IMG / 2));
    for (int i = tid; i < IMG / 16; i += 256) reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(img)[i];
    float* __restrict__ rec = stats + ((size_t)bh * nb64 + blk) * SW;
    if (tid < DV) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < NWV; ++i) t += csum[i][tid];
      rec[tid] = t;
    }
    if (w == NWV % 4) {
      const int nn = lane & 31, h = lane >> 5;
      f32x16 acc = splat16(0.f);
#pragma unroll
      for (int k0 = 0; k0 < BN; k0 += 16) {
        u32 av[4], bv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 8 * h + 2 * i;
          const int c = nn < 16 ? nn : 0;
          const u32 x0 = kl[key * 16 + c], x1 = kl[(key + 1) * 16 + c];
          av[i] = nn < 16 ? (x0 | (x1 << 16)) : 0u;
          bv[i] = nn == 16 ? 0x3f803f80u : av[i];   // bf16 (1, 1)
        }
        acc = mfma32x32x16((u32x4){av[0], av[1], av[2], av[3]}, (u32x4){bv[0], bv[1], bv[2], bv[3]}, acc);
      }
      // lane: column nn, rows c32_row(i, h) (< 16 for i < 8)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int a = c32_row(i, h);
        if (nn < 16 && a <= nn) rec[DV + kStatK2 + 16 * a - a * (a - 1) / 2 + nn - a] = a == nn ? acc[i] : 2.f * acc[i];
        if (nn == 16) rec[DV + kStatK1 + a] = acc[i];
      }
      if (lane < 8) rec[DV + kStatK2 + kTri + lane] = lane == 0 ? (float)eb : 0.f;
    }
  }
}

// stats[bh][blk][sw] -> exclusive prefix over blk, in place, of columns [0, nsum); the columns
// from nsum on (the exponent words) are left alone.  Work-group (bh, g) scans columns
// 16 g .. 16 g + 15 of head bh in tiles of 256 blocks: 16 threads per column each sum a run of 16
// blocks, a 16-term scan of the run totals gives each run's offset, and a carry links the tiles.
// With vt set (the packed parallel pre-pass), one more work-group per head (the last column group
// index) settles the head's V exponent (vt_head_exponent) beside the scans: it reads the block
// exponent words and writes the head's, which no scan touches (columns from nsum on); other users
// scan every column (nsum = sw).
__device__ void vt_head_exponent(float* __restrict__ s, uint16_t* __restrict__ vt, int nb64, int sw, int vt_halves);

__global__ __launch_bounds__(256) void stats_scan_kernel(float* __restrict__ stats, int nb64, int sw, int nsum,
                                                         uint16_t* __restrict__ vt, int vt_halves) {
  constexpr int CW = 16, NT = 256 / CW, TB = 256, PER = TB / NT;
  __shared__ float tile[TB][CW + 1];
  __shared__ float tot[NT][CW];
  if (vt != nullptr && (int)blockIdx.y == (int)gridDim.y - 1) {
    vt_head_exponent(stats + (size_t)blockIdx.x * nb64 * sw + nsum, vt + (size_t)blockIdx.x * nb64 * vt_halves, nb64, sw,
                     vt_halves);
    return;
  }
  const int tid = threadIdx.x, col = tid % CW, g = tid / CW;
  const bool summed = CW * (int)blockIdx.y + col < nsum;
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
      if (bl < nt && summed) s[(size_t)(t0 + bl) * sw + col] = tile[bl][col];
    }
    carry = all;
    __syncthreads();
  }
}

// The head's V exponent E = max_b e_b over its blocks (e[b * sw] = e_b, written by the pack),
// stored in every record (e[b * sw + 1]); blocks with e_b < E have their fp16 V^T multiplied by
// 2^(e_b - E) in place.  Block exponents go through LDS 1024 at a time and each wave tests 64
// of them with one ballot, so a head whose blocks share one exponent costs a few loads.
__device__ void vt_head_exponent(float* __restrict__ e, uint16_t* __restrict__ vt, int nb64, int sw, int vt_halves) {
  constexpr int TB = 1024;
  __shared__ int ex[TB];
  __shared__ int wmax[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int m = -128;
  for (int b = tid; b < nb64; b += 256) m = max(m, (int)e[(size_t)b * sw]);
  m = (int)wave_max_u32((u32)(m + 1024)) - 1024;   // exponents are above -1024
  if (lane == 0) wmax[w] = m;
  __syncthreads();
  const int E = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
  for (int t0 = 0; t0 < nb64; t0 += TB) {
    const int nt = min(TB, nb64 - t0);
    for (int i = tid; i < nt; i += 256) {
      ex[i] = (int)e[(size_t)(t0 + i) * sw];
      e[(size_t)(t0 + i) * sw + 1] = (float)E;
    }
    __syncthreads();
    for (int c0 = 64 * w; c0 < nt; c0 += 256) {
      const bool low = c0 + lane < nt && ex[c0 + lane] < E;
      unsigned long long mask = __ballot(low);
      while (mask != 0ull) {
        const int i = __builtin_ctzll(mask);
        mask &= mask - 1ull;
        const float f = __builtin_ldexpf(1.0f, ex[c0 + i] - E);
        u32x4* blk = reinterpret_cast<u32x4*>(vt + (size_t)(t0 + c0 + i) * vt_halves);
        for (int u = lane; u < vt_halves / 8; u += 64) {
          u32x4 x = blk[u];
#pragma unroll
          for (int j = 0; j < 4; ++j) x[j] = pack_f16x2(f16_lo_to_f32(x[j]) * f, f16_hi_to_f32(x[j]) * f);
          blk[u] = x;
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace la
