// Feature groups and segment sizes shared by the segment-state chunked kernels (bf16 in
// chunked_general.hip, fp32 in chunked_general_f32.hip).
//
// With a' = [scale q, 1] and b' = [k, 1], p(s) = 1 + s + s^2/2 = 1/2 sum_ij a'_i a'_j b'_i b'_j
// + 1/2.  The pairs (i, j) are grouped in 16-wide blocks of j over the dims padded to
// DP = 16 ceil(d/16) plus the augmented index DP (the 1), keeping the upper block triangle, in
// i-major order:
//   quad groups   (i, J)  i < DP, J = i/16 .. DB-1   features a_i a_j, j in block J,
//                                                     weight 1/2 on the diagonal block, 1 above
//   linear groups (DP, J) J < DB                      features a_j,       weight 1
//   constant      (DP, DB)                            feature 1 (j = DP), weight 1
// A query's numerator is sum_f w_f a'_i a'_j T_f with T_f = sum_u b'_i(u) b'_j(u) v_u over the
// earlier segments' tokens, its denominator the same against z_f = sum_u b'_i(u) b'_j(u).
#pragma once

#include <utility>

#include "la_common.hpp"

namespace la {
namespace {

constexpr int GL = 512;    // tokens per segment
constexpr int GC = 64;     // tokens per chunk of the state kernel
constexpr int GQ = 256;    // queries per output work-group

template <int DP>
struct GFeat {
  static constexpr int DB = DP / 16;
  static constexpr int NQ = 8 * DB * (DB + 1);      // quad groups
  static constexpr int NG = NQ + DB + 1;            // + linear + constant
  static constexpr int NGP = (NG + 1) & ~1;         // even: two groups per 32-feature tile
  static constexpr int NT = NGP / 2;                // tiles
  static constexpr int NGB = (NGP + 3) / 4;         // blocks of 4 groups (64 features)
  static constexpr int NWGA = (NGP + 15) / 16;      // state work-groups per head
};

// (i, J) of group g in the i-major order above; the padding group past NG repeats the constant
// group (the output kernel never reads it).
template <int DP>
__device__ __forceinline__ void group_ij(int g, int& i, int& J) {
  constexpr int DB = DP / 16, NQ = GFeat<DP>::NQ;
  if (g < NQ) {
    int start = 0;
#pragma unroll
    for (int I = 0; I < DB; ++I) {
      const int c = DB - I, cnt = 16 * c;
      if (g < start + cnt) {
        const int off = g - start;
        i = 16 * I + off / c;
        J = I + off % c;
        return;
      }
      start += cnt;
    }
  }
  const int r = g - NQ;
  i = DP;
  J = r < DB ? r : DB;
}

template <int DP>
__device__ __forceinline__ float group_weight(int g) {
  if (g >= GFeat<DP>::NG) return 0.f;
  int i, J;
  group_ij<DP>(g, i, J);
  if (i < DP) return J == (i >> 4) ? 0.5f : 1.0f;
  return 1.0f;
}

}  // namespace
}  // namespace la
