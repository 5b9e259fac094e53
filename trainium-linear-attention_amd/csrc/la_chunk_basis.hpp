// Feature basis, workspace records and shared device helpers of the chunked BASED kernels
// (d = 16, based_chunked.hip).  Internal to libbased_la.so.
//
// The basis: 2 p(s) = 2 + 2 s + s^2 = sum_f qf(q~) kf(k~) over 160 feature slots holding the 153
// distinct features of the symmetric Taylor map of benchmarks/chunked_attention_benchmark.py:34-53
// (the constant, q~_i, q~_i^2 and q~_i q~_j for i < j) once each, plus 7 zero slots.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "la_common.hpp"

namespace la {
namespace chunk_basis {

constexpr int CH = 128;         // tokens per chunk
constexpr int NF = 160;         // feature slots
constexpr int QRS = 24;         // row stride (halves) of the q~ / k~ row tables: 48 B
constexpr int KRS = 136;        // row stride (halves) of the K^T and V^T tables: 272 B
constexpr int STS = 168;        // row stride (halves) of S^T: 336 B
constexpr int KT_ROWS = 20;
constexpr int R_ONES = 16, R_ZA = 17, R_ZB = 18, R_TWOS = 19;   // constant rows of K^T: 1/2, 0, 0, 1
constexpr int kNoExp = -1024;   // exponent of an all-zero quantity (below every exponent the kernels form)

// ---- feature templates
//
// Slot f = 16 kk + 8 h + 2 m + e: K-step kk, lane half h, packed register m, half e.  The q side
// of (kk, m) is template tpl(4 kk + m) applied to the register pairs R'_x = R_{(x + 2h) mod 8}
// (and R2' = 2 R'):
//   L a     : R2'_a                       (2 q~_i)
//   S a     : R'_a * R'_a                 (q~_i^2)
//   X a     : R2'_a * swap(R'_a)          (2 q~_2x q~_2x+1 in the low half; the high half
//                                          duplicates it and is unused, except for a = 0 where
//                                          it is replaced by 1: the constant feature)
//   P a b s : R2'_a * (s ? swap(R'_b) : R'_b)
// The rotation by 2h makes every template cover two disjoint sets of registers, so the 40
// templates hold each of the 153 features exactly once.  Templates of one K-step share the
// type and use a = 0, 1, 4, 5, which keeps the k-side row reads of a K-step on distinct LDS
// banks.
enum { TL = 0, TS = 1, TX = 2, TP = 3 };
struct Tpl {
  int t, a, b, sw;
};
__host__ __device__ constexpr Tpl tpl(int i) {
  const int kk = i >> 2, m = i & 3, a = (m & 1) + 4 * (m >> 1);   // 0, 1, 4, 5
  if (kk == 0) return Tpl{TL, a, 0, 0};
  if (kk == 1) return Tpl{TS, a, 0, 0};
  if (kk == 2) return Tpl{TX, a, 0, 0};
  if (kk < 9) return Tpl{TP, a, (a + ((kk - 1) >> 1)) & 7, (kk - 1) & 1};
  return m < 2 ? Tpl{TP, a, a + 4, 0} : Tpl{TP, a, a - 4, 1};   // register pairs 4 apart
}

// k-side rows (K^T table rows multiplied together) of feature slot f.
struct KRows {
  int a, b;
};
__host__ __device__ constexpr KRows krows(int f) {
  const int kk = f >> 4, h = (f >> 3) & 1, m = (f >> 1) & 3, e = f & 1;
  const Tpl t = tpl(4 * kk + m);
  const int x = (t.a + 2 * h) & 7, y = (t.b + 2 * h) & 7;
  if (t.t == TL) return KRows{2 * x + e, R_ONES};
  if (t.t == TS) return KRows{2 * x + e, 2 * x + e};
  if (t.t == TX) {
    if (e == 0) return KRows{2 * x, 2 * x + 1};
    return (t.a == 0 && h == 0) ? KRows{R_TWOS, R_ONES} : KRows{R_ZA, R_ZB};
  }
  return KRows{2 * x + e, t.sw ? 2 * y + 1 - e : 2 * y + e};
}

// Reference feature (benchmarks/chunked_attention_benchmark.py:34-53 order: 1, x_i, x_i^2,
// x_i x_j for i < j row-major) of slot f, and the factor from the k side of 2p (four times the
// table products) to it as an index into {1/2, 1, 1/sqrt 2, 1}; ref = -1 for unused slots.
struct RefFeat {
  int ref, fac;
};
__host__ __device__ constexpr RefFeat ref_feature(int f) {
  const int kk = f >> 4, h = (f >> 3) & 1, m = (f >> 1) & 3, e = f & 1;
  const Tpl t = tpl(4 * kk + m);
  const int x = (t.a + 2 * h) & 7, y = (t.b + 2 * h) & 7;
  int i = 0, j = 0;
  if (t.t == TL) return RefFeat{1 + 2 * x + e, 1};
  if (t.t == TS) return RefFeat{17 + 2 * x + e, 2};
  if (t.t == TX) {
    if (e == 1) return (t.a == 0 && h == 0) ? RefFeat{0, 0} : RefFeat{-1, 0};
    i = 2 * x;
    j = 2 * x + 1;
  } else {
    i = 2 * x + e;
    j = t.sw ? 2 * y + 1 - e : 2 * y + e;
  }
  const int lo = i < j ? i : j, hi = i < j ? j : i;
  return RefFeat{33 + lo * (31 - lo) / 2 + (hi - lo - 1), 3};
}

// Row order of a 32-row MFMA operand whose accumulator is reused as the next operand: C row
// 8 jj + 4 h + i (lane half h) carries item perm32 = 16 (jj >> 1) + 8 h + 4 (jj & 1) + i, so
// lane half h holds items 16 J + 8 h .. +7 in accumulator elements 8 J .. 8 J + 7.
__host__ __device__ constexpr int perm32(int rho) {
  return 16 * (rho >> 4) + 8 * ((rho >> 2) & 1) + 4 * ((rho >> 3) & 1) + (rho & 3);
}

struct ChunkParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  float* state_out;
  uint16_t* wsS;    // [BH][P][64][NF] fp16 S^T increments, then prefixes, in units of 2^wsE / 2^wsEP
  float* wsG;       // [BH][P][64 lanes][16] fp32 Gram increments (accumulator layout), then prefixes
  int* wsE;         // [BH][P] exponent of each increment (slot P - 1: the imported state)
  int* wsEP;        // [BH][P] exponent of each prefix
  int BH, N, dv, P, seg_chunks;
  int ostride;      // increment segments per output segment (the output pass's work-group covers
                    // ostride consecutive segments, starting from the prefix of the first)
  float qs, ks;                      // q~ = qs q (= sqrt(scale) q); K^T table rows ks k = q~-scale k / 2
  float eps;
  float st_fac[4];                   // k side of 2p -> reference feature factors (state export)
  float st_inv[4];                   // their inverses (initial state import)
  const float* state_in;             // optional initial state, reference basis (BH, 153, dv + 1)
  float prev_tokens;                 // tokens summarised by state_in (0 without one)
  float* den_out;                    // optional (BH, N): each row's denominator without eps
  int normalize, out_f32, vec_out;
  // full layer (chunked_layer_kernel): the sliding-window softmax branch's q_sw, k_sw (BH, N, dsw)
  // bf16, its window and scale * log2(e)
  const uint16_t* qsw;
  const uint16_t* ksw;
  int window;
  float sw_log2;
};

__device__ __forceinline__ void map_segment(int wg, int BH, int P, int& bh, int& p) {
  if ((BH & 7) == 0) {
    const int x = wg & 7, slot = wg >> 3;
    const int hx = slot / P;
    p = slot - hx * P;
    bh = hx * 8 + x;
  } else {
    bh = wg / P;
    p = wg - bh * P;
  }
}

constexpr int GRS = 40;   // row stride (halves) of the fp16 Gram matrix in LDS: 80 B

__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); global loads and stores stay in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ u32 swap16(u32 x) { return __builtin_amdgcn_alignbit(x, x, 16); }

// Half index of the 16-byte unit u (tokens 8u .. 8u + 7) of V^T row c.  Rows are 17 units apart
// and row c = 8 j + e (j = c / 8) is stored at row position 8 j + (e ^ (j mod 8)), so unit u of
// row c sits in 16-byte bank group (8 j + (e ^ j) + u) mod 16.  On gfx950 (64 dword banks; as
// measured with SQ_LDS_BANK_CONFLICT):
//   * ds_read_b128 serves a wave in four passes of 16 lanes, lanes l with the same l >> 5 and
//     the same parity of bits 2..4 of l; the MFMA operand reads (lane r reads row 32 n + r at
//     one unit) then take 16 rows in distinct bank groups in every pass;
//   * ds_write_b32 serves 32 lanes per pass over 32 dword banks; the staging stores (rows 8 j + e
//     for j = 0..7 at one e, four token pairs each) land at dword 4 (((e ^ j) + u) mod 8) + t,
//     distinct over j and t.
// A row keeps its units in order, so every read is a per-lane base plus an immediate offset.
__device__ __forceinline__ int vt_row(int c) { return (c & ~7) | ((c ^ (c >> 3)) & 7); }
__device__ __forceinline__ int vt_off(int c, int u) { return vt_row(c) * KRS + 8 * u; }

// Row position of K^T row `row`: rows 8..15 rotated by two within their octet.  The staging
// stores (ds_write_b32, 32 lanes per pass over 32 dword banks) write rows d0 + i for d0 = 0, 4,
// 8, 12 at once, eight token pairs each; rows 8 apart (17 units) would share banks, rotated they
// fill all 32.  The feature reads keep their bank spread (rows 8..15 stay in bank groups 8..15).
__device__ __forceinline__ int kt_row(int row) { return (row & ~7) == 8 ? 8 + ((row + 2) & 7) : row; }

// Constant rows of the K^T table (written once per kernel).
__device__ __forceinline__ void init_kt_constants(uint16_t* KT, int tid, int nthreads) {
  for (int i = tid; i < 4 * (CH / 2); i += nthreads) {
    const int row = R_ONES + (i >> 6), col = 2 * (i & 63);
    const u32 val = row == R_ONES ? 0x38003800u : (row == R_TWOS ? 0x3c003c00u : 0u);
    *reinterpret_cast<u32*>(&KT[row * KRS + col]) = val;
  }
}

// K^T row holding component rho of g_u = [k~_u | 1 | 0 ...] (the Gram operand).
__device__ __forceinline__ int gram_row(int rho) { return rho < 16 ? rho : (rho == 16 ? R_ONES : R_ZA); }

__device__ __forceinline__ u32 swap_quad_pairs(u32 x) {
  // lanes l and l ^ 2 exchange (DPP quad_perm [2, 3, 0, 1])
  return (u32)__builtin_amdgcn_mov_dpp((int)x, 0x4e, 0xf, 0xf, false);
}

// Wave-wide maxima of two 16-bit values at once, packed (hi, lo) into one word: the DPP steps of
// wave_max_u32 on v_pk_max_u16.
__device__ __forceinline__ u32 wave_max_u16x2(u32 x) {
  typedef __attribute__((__vector_size__(2 * sizeof(unsigned short)))) unsigned short u16x2;
  auto step = [](u32 a, u32 b) -> u32 {
    return __builtin_bit_cast(u32, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
  };
  x = step(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false));
  x = step(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false));
  x = step(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false));
  x = step(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false));
  x = step(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false));
  x = step(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false));
  return (u32)__builtin_amdgcn_readlane((int)x, 63);
}

// floor(log2 x) of a positive fp32 magnitude given by its bits; kNoExp for zero.
__device__ __forceinline__ int exp_of_f32bits(u32 b) { return b == 0u ? kNoExp : (int)(b >> 23) - 127; }

// The largest of four per-wave maxima in LDS, as a wave-uniform (scalar) value: every lane
// reads the same words, and readfirstlane tells the compiler so, which keeps the decisions
// taken on it uniform branches.
__device__ __forceinline__ u32 lds_max4(const u32* x) {
  return (u32)__builtin_amdgcn_readfirstlane((int)max(max(x[0], x[1]), max(x[2], x[3])));
}

// Lowest unit of V and the state: every factor 2^-U, 2^(U - U') the kernels form stays finite
// in fp32, and V 2^-U stays in fp16's normal range for every nonzero bf16 v (|v| >= 2^-133).
constexpr int kMinUnit = -126;

// Exponent of the first chunk from floor(log2 max |v|): 0 while max |v| lies in [2^-6, 2^13)
// (V^T is then v itself in fp16, without a multiply), else the one that puts max |v| in
// [2^7, 2^8), at least kMinUnit; an all-zero chunk takes kMinUnit, which the first nonzero V
// raises as far as it needs.
__device__ __forceinline__ int first_unit(int eV) {
  if (eV == kNoExp) return kMinUnit;
  return (eV >= -6 && eV <= 12) ? 0 : max(eV - 7, kMinUnit);
}


// Slot of row r of the update tile of block b.
__device__ __forceinline__ int block_slot(int b, int r) { return 32 * b + perm32(r); }

// Gram coordinate and factor of a K^T row: z_f = fa fb G[da][db] for slot rows (a, b).
__device__ __forceinline__ void kt_row_dim(int row, int& d, float& f) {
  if (row < 16) { d = row; f = 1.f; }
  else if (row == R_ONES) { d = 16; f = 1.f; }
  else if (row == R_TWOS) { d = 16; f = 2.f; }
  else { d = 0; f = 0.f; }
}

}  // namespace chunk_basis
}  // namespace la
