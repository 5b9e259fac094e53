// Global -> register -> LDS staging of 64-key blocks of K (row-major [key][d]) and V
// (transposed [dv][key]) for the bf16 kernels.  The transpose makes the V operand of the
// P.V MFMA (keys contiguous per lane) a pair of 8-byte LDS reads.
#pragma once

#include "la_common.hpp"

namespace la {

constexpr int BN = 64;        // keys per LDS block
constexpr int VROW = BN + 4;  // V^T row stride (bf16): 34 dwords -> conflict-free 8-byte reads

// Global -> register -> LDS staging of one 64-key block of K (row-major) and V (transposed).
// F16V converts V from bf16 to fp16(v 2^vexp) on the way, vexp chosen by the caller from max |v|
// so that the values land in fp16's normal range, so the P.V product can run as an fp16 MFMA.
// The power of two is applied by ldexp on each value, which is exact and stays finite for every
// vexp (a factor 2^vexp would overflow for an all-zero V, whose vexp is 128 and up).
template <int KS, int MT, bool VEC, bool F16V = false>
struct BlockStager {
  static constexpr int DK = 16 * KS, DV = 32 * MT, KROW = DK + 8;
  static constexpr int KCHUNKS = BN * DK / 8;            // 16-byte chunks of the K block
  static constexpr int KPT = (KCHUNKS + 255) / 256;      // per thread
  static constexpr int VGROUPS = (DV / 4) * (BN / 4);    // 4 keys x 4 dv groups
  static constexpr int VPT = (VGROUPS + 255) / 256;
  u32x4 kr[KPT];
  u32x2 vr[VPT][4];
  int vexp = 0;   // F16V: V is stored as fp16(v 2^vexp)

  __device__ __forceinline__ void load(const uint16_t* __restrict__ kg, const uint16_t* __restrict__ vg,
                                       int row0, int N, int d, int dv, int tid) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int c = tid + 256 * r;
      const int key = c / (DK / 8), col = 8 * (c % (DK / 8));
      const int row = row0 + key;
      u32x4 x = {0u, 0u, 0u, 0u};
      if (c < KCHUNKS && row < N) {
        const uint16_t* src = kg + (size_t)row * d + col;
        if (VEC) {
          if (col < d) x = *reinterpret_cast<const u32x4*>(src);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) e[i] = (col + i < d) ? src[i] : (uint16_t)0;
          x = (u32x4){e[0] | ((u32)e[1] << 16), e[2] | ((u32)e[3] << 16), e[4] | ((u32)e[5] << 16),
                      e[6] | ((u32)e[7] << 16)};
        }
      }
      kr[r] = x;
    }
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int g = tid + 256 * r;
      const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
      const int col = 4 * g4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + 4 * kg4 + i;
        u32x2 x = {0u, 0u};
        if (g < VGROUPS && row < N) {
          const uint16_t* src = vg + (size_t)row * dv + col;
          if (VEC) {
            if (col < dv) x = *reinterpret_cast<const u32x2*>(src);
          } else {
            uint16_t e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = (col + t < dv) ? src[t] : (uint16_t)0;
            x = (u32x2){e[0] | ((u32)e[1] << 16), e[2] | ((u32)e[3] << 16)};
          }
        }
        vr[r][i] = x;
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* Ks, uint16_t* VTs, int tid) const {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int c = tid + 256 * r;
      if (c < KCHUNKS) {
        const int key = c / (DK / 8), col = 8 * (c % (DK / 8));
        *reinterpret_cast<u32x4*>(Ks + key * KROW + col) = kr[r];
      }
    }
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int g = tid + 256 * r;
      if (g < VGROUPS) {
        const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
        // vr[r][i] = {v[key i][dv0] | v[key i][dv0+1] << 16, v[key i][dv0+2] | v[key i][dv0+3] << 16}
        const u32 a0 = vr[r][0][0], a1 = vr[r][1][0], a2 = vr[r][2][0], a3 = vr[r][3][0];
        const u32 b0 = vr[r][0][1], b1 = vr[r][1][1], b2 = vr[r][2][1], b3 = vr[r][3][1];
        u32x2 c0, c1, c2, c3;
        if (F16V) {
          const int s = vexp;
          c0 = (u32x2){pack_f16x2(__builtin_ldexpf(bf16_lo_to_f32(a0), s), __builtin_ldexpf(bf16_lo_to_f32(a1), s)),
                       pack_f16x2(__builtin_ldexpf(bf16_lo_to_f32(a2), s), __builtin_ldexpf(bf16_lo_to_f32(a3), s))};
          c1 = (u32x2){pack_f16x2(__builtin_ldexpf(bf16_hi_to_f32(a0), s), __builtin_ldexpf(bf16_hi_to_f32(a1), s)),
                       pack_f16x2(__builtin_ldexpf(bf16_hi_to_f32(a2), s), __builtin_ldexpf(bf16_hi_to_f32(a3), s))};
          c2 = (u32x2){pack_f16x2(__builtin_ldexpf(bf16_lo_to_f32(b0), s), __builtin_ldexpf(bf16_lo_to_f32(b1), s)),
                       pack_f16x2(__builtin_ldexpf(bf16_lo_to_f32(b2), s), __builtin_ldexpf(bf16_lo_to_f32(b3), s))};
          c3 = (u32x2){pack_f16x2(__builtin_ldexpf(bf16_hi_to_f32(b0), s), __builtin_ldexpf(bf16_hi_to_f32(b1), s)),
                       pack_f16x2(__builtin_ldexpf(bf16_hi_to_f32(b2), s), __builtin_ldexpf(bf16_hi_to_f32(b3), s))};
        } else {
          c0 = (u32x2){(a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16)};
          c1 = (u32x2){(a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u)};
          c2 = (u32x2){(b0 & 0xffffu) | (b1 << 16), (b2 & 0xffffu) | (b3 << 16)};
          c3 = (u32x2){(b0 >> 16) | (b1 & 0xffff0000u), (b2 >> 16) | (b3 & 0xffff0000u)};
        }
        uint16_t* dst = VTs + (4 * g4) * VROW + 4 * kg4;
        *reinterpret_cast<u32x2*>(dst) = c0;
        *reinterpret_cast<u32x2*>(dst + VROW) = c1;
        *reinterpret_cast<u32x2*>(dst + 2 * VROW) = c2;
        *reinterpret_cast<u32x2*>(dst + 3 * VROW) = c3;
      }
    }
  }
};

// 16-byte fragment of a bf16 row: elements [col, col + 8), zero past `len` or when the row is
// out of range.  VEC selects one vector load (len % 8 == 0, 16-byte aligned rows).
template <bool VEC>
__device__ __forceinline__ u32x4 load_row8(const uint16_t* __restrict__ rowp, int col, int len, bool valid) {
  u32x4 x = {0u, 0u, 0u, 0u};
  if (!valid) return x;
  if (VEC) {
    if (col < len) x = *reinterpret_cast<const u32x4*>(rowp + col);
  } else {
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (col + i < len) ? rowp[col + i] : (uint16_t)0;
    x = (u32x4){e[0] | ((u32)e[1] << 16), e[2] | ((u32)e[3] << 16), e[4] | ((u32)e[5] << 16),
                e[6] | ((u32)e[7] << 16)};
  }
  return x;
}

// Stores 4 consecutive output values of row `obase` starting at `col` (bounds-checked by dv),
// plus the same elements of `addend` (fp32, same layout as the output) when it is not null.
// Each element of addend is read by the thread that then writes it, so addend may be the output.
template <bool VEC>
__device__ __forceinline__ void store_out4(void* out, bool out_f32, size_t obase, int col, int dv, const float* y_in,
                                           const float* addend = nullptr) {
  float y[4] = {y_in[0], y_in[1], y_in[2], y_in[3]};
  if (addend != nullptr) {
    if (VEC) {
      if (col < dv) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(addend + obase + col);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] += a[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < dv) y[e] += addend[obase + col + e];
    }
  }
  if (VEC) {
    if (col < dv) {
      if (out_f32)
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + obase + col) = (f32x4){y[0], y[1], y[2], y[3]};
      else
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + obase + col) =
            (u32x2){pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (col + e < dv) {
        if (out_f32)
          static_cast<float*>(out)[obase + col + e] = y[e];
        else
          static_cast<uint16_t*>(out)[obase + col + e] = f32_to_bf16_bits(y[e]);
      }
    }
  }
}

}  // namespace la
