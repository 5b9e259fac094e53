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
// rows are d = 16 bf16 (16-byte aligned), v rows dv % 8 == 0 bf16 (8-byte aligned).  Loads go
// through raw buffer resources over the head's rows, so rows past N (and columns past dv) read
// as zero without per-lane branches.  Per block:
//  * V^T: thread t takes keys 2 (t / CPR) and 2 (t / CPR) + 1, columns 8 (t % CPR) .. +7, so it
//    holds both halves of 8 fp16 pairs of the transposed block; it writes them into an LDS
//    image of the block (padding zero), which whole-chunk stores then copy out;
//  * column sums of V from the same registers: a butterfly over the lanes of one column group
//    (each exchange halves the columns a lane carries, 7 shuffles for 8 columns), then the
//    waves through LDS;
//  * k sums and the k k^T triangle from one 32x32x16 MFMA chain over the 64 keys (wave
//    NWV % 4, first, beside the other waves' V conversion): A = K^T (rows 16..31 zero), B = K
//    with a column of ones at 16, so C[a][b] = (k k^T)[a][b] and C[a][16] = k1[a]; K^T sits in
//    LDS as rows of keys, so each operand is one 16-byte read.
constexpr int PPW = 1;   // blocks per pack work-group
constexpr int KTS = BN + 8;   // K^T row stride (halves): 144 bytes, the operand reads on distinct banks

template <int DV, int ROW>
__global__ __launch_bounds__(256) void par_pack_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                       uint16_t* __restrict__ vt, float* __restrict__ stats, int N,
                                                       int dv, int nb64) {
  constexpr int SW = stats_width(DV);
  constexpr int CPR = DV / 8;                 // 8-element column groups per V row
  constexpr int NT = (BN / 2) * CPR;          // threads holding a (key pair, column group)
  constexpr int NWV = NT / 64;                // waves among them
  constexpr int IMG = VtBlock<DV, ROW>::bytes;
  static_assert(ROW % 2 == 0 && NT <= 256 && (CPR == 4 || CPR == 8), "pack layout");
  __shared__ __attribute__((aligned(16))) u32 img[IMG / 4];
  __shared__ __attribute__((aligned(16))) uint16_t kt[16 * KTS];
  __shared__ float csum[NWV][DV];
  __shared__ u32 vmx[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bh = blockIdx.y, blk0 = blockIdx.x * PPW;
  const int nb = min(PPW, nb64 - blk0);
  const int kp = tid / CPR, cg = tid % CPR, col = 8 * cg;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(v + (size_t)bh * N * dv, (u32)N * (u32)dv * 2u);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(k + (size_t)bh * N * 16, (u32)N * 32u);

  for (int i = tid; i < IMG / 16; i += 256) reinterpret_cast<u32x4*>(img)[i] = (u32x4){0u, 0u, 0u, 0u};

  u32x4 va[PPW], vb[PPW], kx[PPW];
#pragma unroll
  for (int b = 0; b < PPW; ++b) {
    const int row0 = (blk0 + b) * BN;
    // rows past N read zero through the resource; threads past NT and columns past dv read
    // nothing (an offset out of range)
    const int vo = (b < nb && tid < NT && col < dv) ? ((row0 + 2 * kp) * dv + col) * 2 : kOffOutOfRange;
    const u32x2 a0 = buf_load_b64(rv, vo), a1 = buf_load_b64(rv, vo + 8);
    const u32x2 b0 = buf_load_b64(rv, vo + 2 * dv), b1 = buf_load_b64(rv, vo + 2 * dv + 8);
    va[b] = (u32x4){a0[0], a0[1], a1[0], a1[1]};
    vb[b] = (u32x4){b0[0], b0[1], b1[0], b1[1]};
    kx[b] = buf_load_b128(rk, (b < nb && tid < 128) ? (row0 + (tid >> 1)) * 32 + 16 * (tid & 1) : kOffOutOfRange);
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
    // K^T: thread t < 128 holds dims 8 (t & 1) .. +7 of key t / 2
    if (tid < 128) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kt[(8 * (tid & 1) + 2 * j) * KTS + (tid >> 1)] = (uint16_t)(kx[b][j] & 0xffffu);
        kt[(8 * (tid & 1) + 2 * j + 1) * KTS + (tid >> 1)] = (uint16_t)(kx[b][j] >> 16);
      }
    }
    __syncthreads();   // image zeroed / the previous block's readers done / maxima and K^T written
    // fp16(v 2^-eb) by ldexp on each value: exact, and finite for an all-zero block (eb = -128)
    const int eb = vexp_step(max(max(vmx[0], vmx[1]), max(vmx[2], vmx[3])) << 16);
    float* __restrict__ rec = stats + ((size_t)bh * nb64 + blk) * SW;
    // k k^T and the k-sums first, so that the record's last writes do not wait for the V^T copy
    if (w == NWV % 4) {
      const int nn = lane & 31, h = lane >> 5;
      f32x16 acc = splat16(0.f);
#pragma unroll
      for (int k0 = 0; k0 < BN; k0 += 16) {
        const u32x4 x = nn < 16 ? *reinterpret_cast<const u32x4*>(&kt[nn * KTS + k0 + 8 * h]) : (u32x4){0u, 0u, 0u, 0u};
        const u32 one = nn == 16 ? 0x3f803f80u : 0u;   // bf16 (1, 1)
        acc = mfma32x32x16(x, nn < 16 ? x : (u32x4){one, one, one, one}, acc);
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
    float part[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const u32 a0 = va[b][e >> 1], a1 = vb[b][e >> 1];
      const float f0 = (e & 1) ? bf16_hi_to_f32(a0) : bf16_lo_to_f32(a0);
      const float f1 = (e & 1) ? bf16_hi_to_f32(a1) : bf16_lo_to_f32(a1);
      part[e] = f0 + f1;   // zero for threads past NT (they loaded nothing)
      if (tid < NT)
        img[(col + e) * (ROW / 2) + kp] = pack_f16x2(__builtin_ldexpf(f0, -eb), __builtin_ldexpf(f1, -eb));
    }
    // column sums over the lanes of this column group (lane bits log2(CPR) .. 5): each exchange
    // keeps the half of the lane's columns that its bit selects and adds the partner's copy of
    // them, so that after three exchanges a lane holds one column's sum over 8 lanes (CPR = 8);
    // with CPR = 4 a fourth exchange adds the other half of the wave
    float p4[4], p2[2];
    {
      const bool up = (lane & CPR) != 0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p4[i] = (up ? part[4 + i] : part[i]) + __shfl_xor(up ? part[i] : part[4 + i], CPR);
    }
    {
      const bool up = (lane & (2 * CPR)) != 0;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        p2[i] = (up ? p4[2 + i] : p4[i]) + __shfl_xor(up ? p4[i] : p4[2 + i], 2 * CPR);
    }
    float p1;
    {
      const bool up = (lane & (4 * CPR)) != 0;
      p1 = (up ? p2[1] : p2[0]) + __shfl_xor(up ? p2[0] : p2[1], 4 * CPR);
    }
    if (CPR == 4) p1 += __shfl_xor(p1, 32);
    // lane's column: col + 4 (bit CPR) + 2 (bit 2 CPR) + (bit 4 CPR)
    const int sc = col + ((lane & CPR) ? 4 : 0) + ((lane & (2 * CPR)) ? 2 : 0) + ((lane & (4 * CPR)) ? 1 : 0);
    if (w < NWV && (CPR == 8 || lane < 32)) csum[w][sc] = p1;
    __syncthreads();
    u32* dst = reinterpret_cast<u32*>(vt + ((size_t)bh * nb64 + blk) * (IMG / 2));
    for (int i = tid; i < IMG / 16; i += 256) reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(img)[i];
    if (tid < DV) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < NWV; ++i) t += csum[i][tid];
      rec[tid] = t;
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
