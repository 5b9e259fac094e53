// Chunked recurrent BASED attention for gfx950 (d = 16, dv <= 64).
//
// Replaces the NKI chunked kernel (kernels/nki_attention_chunked.py:27-113) and the feature
// map + padding of its wrapper (benchmarks/chunked_attention_benchmark.py:96-126).  The
// recurrence is the reference's: per chunk c,
//     out_c = phi(Q_c) S + causal(phi(Q_c) phi(K_c)^T) V_c,    S += phi(K_c)^T V_c,
// extended with the K-sum z (den = phi(q).z + intra row sum) so it can also normalise.
//
// Design for MI355X:
//   * Every product runs on v_mfma_f32_32x32x16_f16 (the 16x16x32 forms issue at half the
//     rate on gfx950).  Chunks are 128 tokens; wave w of a work-group owns query tokens
//     32w .. 32w+31 of every chunk.
//   * phi is never materialised in HBM.  With q~ = alpha q and k~ = beta k (alpha beta = scale)
//     the kernel works in units of 2p:  2 p(s) = 2 + 2 s + s^2 = sum_f qf(q~) kf(k~), over 160
//     feature slots (10 K-steps of 16) holding the 153 distinct features of the symmetric
//     Taylor map: the constant, q~_i, q~_i^2 and q~_i q~_j (i < j).  The q side of a K-step is
//     four packed-fp16 products of q~'s eight register pairs R_x = (q~_2x, q~_2x+1); the two
//     lane halves of the MFMA operand hold q~ rotated by one register, so one v_pk_mul_f16
//     yields two features for each half ("templates" below).  All coefficients live on the k
//     side, which multiplies two rows of an LDS table [k~ | 2 k~ | 1 | 0 | 2] (K^T, token pairs
//     packed), again one v_pk_mul_f16 per two products.
//   * The state S (160 x dv, fp32 MFMA accumulators) stays in registers across chunks,
//     partitioned over the waves by blocks of 32 features; every chunk it is published to LDS
//     as fp16 S^T for the inter-chunk product phi(Q) S of all waves.
//   * The k-sums z of all 153 features follow from the Gram matrix G = sum_u g_u g_u^T of
//     g_u = [k~_u | 1] (17 x 17, one 32 x 32 accumulator, 8 MFMAs per chunk): the denominator of
//     the earlier tokens is q'^T G q' + count with q' = [q~ | 1], two MFMAs per query tile.
//   * Intra-chunk: scores 1 + q~.k~ on the same fp16 q~, k~ (one MFMA per 32 x 32 tile),
//     P = b^2 + 1 = 2 p, masked on the diagonal tile, then P V on MFMA.  The score tile's key
//     rows are permuted so that its accumulator layout is directly the B operand of P V.
//   * Sequence parallelism: the sequence is cut into P segments of whole chunks.  Kernel 1
//     computes every segment's state increment (fp16 S^T, fp32 G) into the workspace, kernel 2
//     turns them into exclusive prefixes, kernel 3 runs the chunk recurrence of all segments
//     in parallel from those prefixes.
#include <math.h>

#include "../../include/based_la.h"
#include "la_common.hpp"
#include "la_internal.hpp"

namespace la {

namespace {

constexpr int CH = 128;         // tokens per chunk
constexpr int NF = 160;         // feature slots
constexpr int QRS = 24;         // row stride (halves) of the q~ / k~ row tables: 48 B
constexpr int KRS = 136;        // row stride (halves) of the K^T and V^T tables: 272 B
constexpr int STS = 168;        // row stride (halves) of S^T: 336 B
constexpr int KT_ROWS = 36;
constexpr int R_ONES = 32, R_ZA = 33, R_ZB = 34, R_TWOS = 35;   // constant rows of K^T
constexpr int NWAVE_OUT = 4;
constexpr int NWAVE_SEG = 5;
constexpr int MAX_SEG = 32;

// ---- feature templates
//
// Slot f = 16 kk + 8 h + 2 m + e: K-step kk, lane half h, packed register m, half e.  The q side
// of (kk, m) is template tpl(4 kk + m) applied to the register pairs R'_x = R_{(x + h) mod 8}:
//   L a     : R'_a                        (q~_i)
//   S a     : R'_a * R'_a                 (q~_i^2)
//   X a     : R'_a * swap(R'_a)           (q~_2x q~_2x+1 in the low half; the high half
//                                          duplicates it and is unused, except for a = 0 where
//                                          it is replaced by 1: the constant feature)
//   P a b s : R'_a * (s ? swap(R'_b) : R'_b)
// The rotation by h makes every template cover two disjoint sets of registers, so the 40
// templates hold each of the 153 features exactly once.  Templates of one K-step share the
// type and use a = 0, 2, 4, 6, which keeps the k-side row reads of a K-step on distinct LDS
// banks.
enum { TL = 0, TS = 1, TX = 2, TP = 3 };
struct Tpl {
  int t, a, b, sw;
};
__host__ __device__ constexpr Tpl tpl(int i) {
  const int kk = i >> 2, m = i & 3, a = 2 * m;
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
  const int x = (t.a + h) & 7, y = (t.b + h) & 7;
  if (t.t == TL) return KRows{16 + 2 * x + e, R_ONES};
  if (t.t == TS) return KRows{2 * x + e, 2 * x + e};
  if (t.t == TX) {
    if (e == 0) return KRows{2 * x, 16 + 2 * x + 1};
    return (t.a == 0 && h == 0) ? KRows{R_TWOS, R_ONES} : KRows{R_ZA, R_ZB};
  }
  return KRows{2 * x + e, 16 + (t.sw ? 2 * y + 1 - e : 2 * y + e)};
}

// Reference feature (benchmarks/chunked_attention_benchmark.py:34-53 order: 1, x_i, x_i^2,
// x_i x_j for i < j row-major) of slot f, and the factor from the internal k side to it as
// an index into {1/2, 2^(sigma/2)/2, 2^sigma/sqrt 2, 2^sigma/2}; ref = -1 for unused slots.
struct RefFeat {
  int ref, fac;
};
__host__ __device__ constexpr RefFeat ref_feature(int f) {
  const int kk = f >> 4, h = (f >> 3) & 1, m = (f >> 1) & 3, e = f & 1;
  const Tpl t = tpl(4 * kk + m);
  const int x = (t.a + h) & 7, y = (t.b + h) & 7;
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
  uint16_t* wsS;    // [BH][P][64][NF] fp16 S^T increments, then prefixes
  float* wsG;       // [BH][P][64 lanes][16] fp32 Gram increments (accumulator layout), then prefixes
  int BH, N, dv, P, seg_chunks;
  float alpha, beta;                 // q~ = alpha q, k~ = beta k
  float eps;
  float st_fac[4];                   // internal -> reference feature factors (state export)
  int normalize, out_f32, vec_out;
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

// LDS image of one chunk and of the published state.
struct OutLds {
  uint16_t Q0[CH * QRS];        // q~ rows (fp16)
  uint16_t Q1[CH * QRS];        // q~ rows rotated left by two elements
  uint16_t Kr[CH * QRS];        // k~ rows
  uint16_t KT[KT_ROWS * KRS];   // k~^T, (2 k~)^T, constant rows
  uint16_t VT[64 * KRS];        // V^T
  uint16_t ST[64 * STS];        // S^T (feature slots)
  uint16_t G16[32 * GRS];       // Gram matrix [k~ | 1]^T [k~ | 1] of earlier tokens, (16,16) zeroed
};
struct SegTables {
  uint16_t KT[KT_ROWS * KRS];
  uint16_t VT[64 * KRS];
};
struct SegLds {
  SegTables buf[2];
};

__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); global loads and stores stay in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ u32 swap16(u32 x) { return __builtin_amdgcn_alignbit(x, x, 16); }

// Constant rows of the K^T table (written once per kernel).
__device__ __forceinline__ void init_kt_constants(uint16_t* KT, int tid, int nthreads) {
  for (int i = tid; i < 4 * (CH / 2); i += nthreads) {
    const int row = R_ONES + (i >> 6), col = 2 * (i & 63);
    const u32 val = row == R_ONES ? 0x3c003c00u : (row == R_TWOS ? 0x40004000u : 0u);
    *reinterpret_cast<u32*>(&KT[row * KRS + col]) = val;
  }
}

// K^T row holding component rho of g_u = [k~_u | 1 | 0 ...] (the Gram operand).
__device__ __forceinline__ int gram_row(int rho) { return rho < 16 ? rho : (rho == 16 ? R_ONES : R_ZA); }

// ---- staging: global -> registers -> (convert) -> LDS
//
// Wave wv (0..3) stages q, k dims 4 wv .. +3 and v dims 16 wv .. +15; lane l the token pair
// 2l, 2l + 1 of the chunk, so that every LDS store instruction writes consecutive dwords of one
// table row.
struct StageRegs {
  u32x2 q[2], k[2];
  u32x4 v[2][2];
};

template <bool VEC_V, bool WITH_Q>
__device__ __forceinline__ void stage_load(StageRegs& s, const ChunkParams& p, const uint16_t* qh,
                                           const uint16_t* kh, const uint16_t* vh, int row0, int l, int wv) {
  const int N = p.N, dv = p.dv;
  const u32 rem = (u32)(N - row0);   // > 0
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kh + (size_t)row0 * 16, rem * 32u);
  __amdgpu_buffer_rsrc_t rq = rk;
  if (WITH_Q) rq = make_rsrc(qh + (size_t)row0 * 16, rem * 32u);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int voff = (2 * l + j) * 32 + 8 * wv;
    if (WITH_Q) s.q[j] = buf_load_b64(rq, voff);
    s.k[j] = buf_load_b64(rk, voff);
  }
  if (VEC_V) {
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vh + (size_t)row0 * dv, rem * (u32)dv * 2u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int hv = 0; hv < 2; ++hv) {
        const int col = 16 * wv + 8 * hv;
        const int voff = col < dv ? ((2 * l + j) * dv + col) * 2 : kOffOutOfRange;
        s.v[j][hv] = buf_load_b128(rv, voff);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = row0 + 2 * l + j;
#pragma unroll
      for (int hv = 0; hv < 2; ++hv) {
        const int col = 16 * wv + 8 * hv;
        uint16_t e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = (row < N && col + i < dv) ? vh[(size_t)row * dv + col + i] : (uint16_t)0;
        s.v[j][hv] = (u32x4){e[0] | ((u32)e[1] << 16), e[2] | ((u32)e[3] << 16), e[4] | ((u32)e[5] << 16),
                             e[6] | ((u32)e[7] << 16)};
      }
    }
  }
}

// Converted staging values of one thread: fp16 q~ / k~ row pieces, k~ and 2 k~ token pairs of
// dims 4 wv + i, V^T token pairs of dims 16 wv + 2 i (+1).
struct StageConv {
  u32 q[2][2], kr[2][2];
  u32 kt[4], kt2[4];
  u32 vt[16];
};

template <bool WITH_Q>
__device__ __forceinline__ void stage_convert(const StageRegs& s, StageConv& o, float alpha, float beta) {
  if (WITH_Q) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      o.q[j][0] = pack_f16x2(alpha * bf16_lo_to_f32(s.q[j][0]), alpha * bf16_hi_to_f32(s.q[j][0]));
      o.q[j][1] = pack_f16x2(alpha * bf16_lo_to_f32(s.q[j][1]), alpha * bf16_hi_to_f32(s.q[j][1]));
    }
  }
  float kf[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    kf[j][0] = beta * bf16_lo_to_f32(s.k[j][0]);
    kf[j][1] = beta * bf16_hi_to_f32(s.k[j][0]);
    kf[j][2] = beta * bf16_lo_to_f32(s.k[j][1]);
    kf[j][3] = beta * bf16_hi_to_f32(s.k[j][1]);
    if (WITH_Q) {
      o.kr[j][0] = pack_f16x2(kf[j][0], kf[j][1]);
      o.kr[j][1] = pack_f16x2(kf[j][2], kf[j][3]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o.kt[i] = pack_f16x2(kf[0][i], kf[1][i]);   // (token 2l, token 2l+1) of dim 4wv+i
    o.kt2[i] = pk_mul_f16(o.kt[i], 0x40004000u);
  }
#pragma unroll
  for (int hv = 0; hv < 2; ++hv) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32 a = s.v[0][hv][w], b = s.v[1][hv][w];
      o.vt[2 * (4 * hv + w)] = pack_f16x2(bf16_lo_to_f32(a), bf16_lo_to_f32(b));
      o.vt[2 * (4 * hv + w) + 1] = pack_f16x2(bf16_hi_to_f32(a), bf16_hi_to_f32(b));
    }
  }
}

// Keeps the conversion above this point (the compiler would otherwise sink it next to the LDS
// stores, between two barriers where every wave waits for it).
template <bool WITH_Q>
__device__ __forceinline__ void stage_pin(StageConv& o) {
  if (WITH_Q) {
#pragma unroll
    for (int j = 0; j < 2; ++j) asm volatile("" : "+v"(o.q[j][0]), "+v"(o.q[j][1]), "+v"(o.kr[j][0]), "+v"(o.kr[j][1]));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(o.kt[i]), "+v"(o.kt2[i]));
#pragma unroll
  for (int i = 0; i < 16; i += 4) asm volatile("" : "+v"(o.vt[i]), "+v"(o.vt[i + 1]), "+v"(o.vt[i + 2]), "+v"(o.vt[i + 3]));
}

template <bool WITH_Q>
__device__ __forceinline__ void stage_write(const StageConv& o, uint16_t* Q0, uint16_t* Q1, uint16_t* Kr,
                                            uint16_t* KT, uint16_t* VT, int l, int wv) {
  const int dq = wv;
  if (WITH_Q) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int tok = 2 * l + j;
      *reinterpret_cast<u32x2*>(&Q0[tok * QRS + 4 * dq]) = (u32x2){o.q[j][0], o.q[j][1]};
      // rotated copy: element i of Q1 is element (i + 2) mod 16 of q~
      *reinterpret_cast<u32*>(&Q1[tok * QRS + ((4 * dq + 14) & 15)]) = o.q[j][0];
      *reinterpret_cast<u32*>(&Q1[tok * QRS + 4 * dq]) = o.q[j][1];
      *reinterpret_cast<u32x2*>(&Kr[tok * QRS + 4 * dq]) = (u32x2){o.kr[j][0], o.kr[j][1]};
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *reinterpret_cast<u32*>(&KT[(4 * dq + i) * KRS + 2 * l]) = o.kt[i];
    *reinterpret_cast<u32*>(&KT[(16 + 4 * dq + i) * KRS + 2 * l]) = o.kt2[i];
  }
  // V^T: row c = 16 dq + 2 i (+1), token pair l
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    *reinterpret_cast<u32*>(&VT[(16 * dq + 2 * i) * KRS + 2 * l]) = o.vt[2 * i];
    *reinterpret_cast<u32*>(&VT[(16 * dq + 2 * i + 1) * KRS + 2 * l]) = o.vt[2 * i + 1];
  }
}

// ---- state update of NB blocks of 32 feature slots over one chunk (all dv)
//
// A = phi(K)^T tile (32 slots x 16 tokens): lane (row r, tokens 8h .. +7 of the K-step) forms
// its slot's product of two K^T rows; B = V (16 tokens x 32 dv) from V^T.
template <int NB>
__device__ __forceinline__ void update_blocks(const uint16_t* KT, const uint16_t* VT, f32x16 (&S)[NB][2],
                                              const int (&ra)[NB], const int (&rb)[NB], int r, int h) {
#pragma unroll
  for (int s = 0; s < CH / 16; ++s) {
    u32x4 bv[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) bv[n] = *reinterpret_cast<const u32x4*>(&VT[(32 * n + r) * KRS + 16 * s + 8 * h]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(&KT[ra[b] + 16 * s + 8 * h]);
      const u32x4 y = *reinterpret_cast<const u32x4*>(&KT[rb[b] + 16 * s + 8 * h]);
      u32x4 a;
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = pk_mul_f16(x[i], y[i]);
#pragma unroll
      for (int n = 0; n < 2; ++n) S[b][n] = mfma32x32x16_f16(a, bv[n], S[b][n]);
    }
  }
}

// Gram matrix G += sum_u g_u g_u^T over the K-steps s of the chunk with (s % step) == first.
__device__ __forceinline__ void gram_update(const uint16_t* KT, f32x16& G, int grow, int h, int first, int step) {
  for (int s = first; s < CH / 16; s += step) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(&KT[grow + 16 * s + 8 * h]);
    G = mfma32x32x16_f16(x, x, G);
  }
}

// Slot of row r of the update tile of block b.
__device__ __forceinline__ int block_slot(int b, int r) { return 32 * b + perm32(r); }

// Gram coordinate and factor of a K^T row: z_f = fa fb G[da][db] for slot rows (a, b).
__device__ __forceinline__ void kt_row_dim(int row, int& d, float& f) {
  if (row < 16) { d = row; f = 1.f; }
  else if (row < 32) { d = row - 16; f = 2.f; }
  else if (row == R_ONES) { d = 16; f = 1.f; }
  else if (row == R_TWOS) { d = 16; f = 2.f; }
  else { d = 0; f = 0.f; }
}

// -------------------------------------------------------------------------------------------
// Kernel 1: state increment of every segment but the last.  Work-group (head, segment); wave w
// owns feature block w (all dv) and K-steps w, w + 5 of the Gram matrix; waves 0..3 stage.
template <bool VEC_V>
__global__ __launch_bounds__(64 * NWAVE_SEG) void chunked_segment_kernel(const ChunkParams p) {
  __shared__ __attribute__((aligned(16))) SegLds L;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  int bh, seg;
  map_segment(blockIdx.x, p.BH, p.P - 1, bh, seg);
  const size_t hrow = (size_t)bh * p.N;
  const uint16_t* kh = p.k + hrow * 16;
  const uint16_t* vh = p.v + hrow * p.dv;
  const int c0 = seg * p.seg_chunks, nch = p.seg_chunks;
  const bool stager = w < 4;

  const KRows kr = krows(block_slot(w, r));
  const int ra[1] = {kr.a * KRS}, rb[1] = {kr.b * KRS};
  const int grow = gram_row(r) * KRS;
  f32x16 S[1][2] = {{splat16(0.f), splat16(0.f)}};
  f32x16 G = splat16(0.f);

  init_kt_constants(L.buf[0].KT, tid, 64 * NWAVE_SEG);
  init_kt_constants(L.buf[1].KT, tid, 64 * NWAVE_SEG);
  StageRegs st;
  StageConv cv;
  if (stager) {
    stage_load<VEC_V, false>(st, p, nullptr, kh, vh, c0 * CH, lane, w);
    stage_convert<false>(st, cv, p.alpha, p.beta);
    stage_write<false>(cv, nullptr, nullptr, nullptr, L.buf[0].KT, L.buf[0].VT, lane, w);
  }
  lds_barrier();
  for (int c = 0; c < nch; ++c) {
    const SegTables& T = L.buf[c & 1];
    if (stager && c + 1 < nch) stage_load<VEC_V, false>(st, p, nullptr, kh, vh, (c0 + c + 1) * CH, lane, w);
    update_blocks<1>(T.KT, T.VT, S, ra, rb, r, h);
    gram_update(T.KT, G, grow, h, w, NWAVE_SEG);
    if (stager && c + 1 < nch) {
      SegTables& U = L.buf[(c + 1) & 1];
      stage_convert<false>(st, cv, p.alpha, p.beta);
      stage_pin<false>(cv);
      stage_write<false>(cv, nullptr, nullptr, nullptr, U.KT, U.VT, lane, w);
    }
    lds_barrier();
  }
  // increment: S^T fp16 [dv][slot]; Gram partials of the waves summed through LDS
  const size_t slot = (size_t)bh * p.P + seg;
  uint16_t* ws = p.wsS + slot * (64 * NF);
#pragma unroll
  for (int n = 0; n < 2; ++n) {
#pragma unroll
    for (int J = 0; J < 2; ++J) {
      const f32x16& a = S[0][n];
      const u32x4 pk = {pack_f16x2(a[8 * J + 0], a[8 * J + 1]), pack_f16x2(a[8 * J + 2], a[8 * J + 3]),
                        pack_f16x2(a[8 * J + 4], a[8 * J + 5]), pack_f16x2(a[8 * J + 6], a[8 * J + 7])};
      *reinterpret_cast<u32x4*>(&ws[(32 * n + r) * NF + 32 * w + 16 * J + 8 * h]) = pk;
    }
  }
  float* red = reinterpret_cast<float*>(&L);   // 5 x 64 x 16 floats = 20 KB, tables no longer read
#pragma unroll
  for (int e = 0; e < 16; e += 4)
    *reinterpret_cast<f32x4*>(&red[(w * 64 + lane) * 16 + e]) = (f32x4){G[e], G[e + 1], G[e + 2], G[e + 3]};
  lds_barrier();
  if (w == 0) {
    float* gout = p.wsG + slot * 1024 + lane * 16;
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
      f32x4 acc = *reinterpret_cast<const f32x4*>(&red[lane * 16 + e]);
#pragma unroll
      for (int ww = 1; ww < NWAVE_SEG; ++ww) acc += *reinterpret_cast<const f32x4*>(&red[(ww * 64 + lane) * 16 + e]);
      *reinterpret_cast<f32x4*>(&gout[e]) = acc;
    }
  }
}

// -------------------------------------------------------------------------------------------
// Kernel 2: exclusive prefixes over segments, in place: afterwards slot p - 1 holds the sum of
// the increments of segments 0 .. p-1.  Thread (head, 16-byte unit); fp32 accumulation.
__global__ __launch_bounds__(256) void chunked_prefix_kernel(const ChunkParams p) {
  constexpr int US = 64 * NF / 8, UG = 1024 / 4;   // 16-byte units of S^T (fp16) and G (fp32)
  const int e = blockIdx.x * 256 + threadIdx.x, bh = blockIdx.y;
  const int nseg = p.P - 1;
  if (e < US) {
    uint16_t* base = p.wsS + (size_t)bh * p.P * (64 * NF) + 8 * (size_t)e;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nseg; s0 += 8) {
      u32x4 x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        x[i] = s0 + i < nseg ? *reinterpret_cast<const u32x4*>(base + (size_t)(s0 + i) * (64 * NF))
                             : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (s0 + i >= nseg) break;
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[2 * j] += f16_lo_to_f32(x[i][j]);
          acc[2 * j + 1] += f16_hi_to_f32(x[i][j]);
          o[j] = pack_f16x2(acc[2 * j], acc[2 * j + 1]);
        }
        *reinterpret_cast<u32x4*>(base + (size_t)(s0 + i) * (64 * NF)) = o;
      }
    }
  } else if (e < US + UG) {
    float* base = p.wsG + (size_t)bh * p.P * 1024 + 4 * (size_t)(e - US);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nseg; s0 += 8) {
      f32x4 x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        x[i] = s0 + i < nseg ? *reinterpret_cast<const f32x4*>(base + (size_t)(s0 + i) * 1024)
                             : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (s0 + i >= nseg) break;
        acc += x[i];
        *reinterpret_cast<f32x4*>(base + (size_t)(s0 + i) * 1024) = acc;
      }
    }
  }
}

// -------------------------------------------------------------------------------------------
// Kernel 3: outputs.  Work-group (head, segment), 4 waves; wave W owns query tokens 32W .. +31
// of each chunk and state blocks {0, 1} (W = 0) or {W + 1}; wave 1 also keeps the Gram matrix.
template <int W>
struct OwnedBlocks {
  static constexpr int NB = W == 0 ? 2 : 1;
  static constexpr int first = W == 0 ? 0 : W + 1;
};
constexpr int kGramWave = 1;

template <int NB>
__device__ __forceinline__ void publish_state(OutLds& L, const f32x16 (&S)[NB][2], int first, int r, int h) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int blk = first + b;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
#pragma unroll
      for (int J = 0; J < 2; ++J) {
        const f32x16& a = S[b][n];
        const u32x4 pk = {pack_f16x2(a[8 * J + 0], a[8 * J + 1]), pack_f16x2(a[8 * J + 2], a[8 * J + 3]),
                          pack_f16x2(a[8 * J + 4], a[8 * J + 5]), pack_f16x2(a[8 * J + 6], a[8 * J + 7])};
        *reinterpret_cast<u32x4*>(&L.ST[(32 * n + r) * STS + 32 * blk + 16 * J + 8 * h]) = pk;
      }
    }
  }
}

// fp16 Gram matrix for the denominator, with the token count G(16,16) left out (it is added
// exactly).  Lane (col j = r, rows 8 jj + 4 h + i) writes row j by symmetry.
__device__ __forceinline__ void publish_gram(OutLds& L, const f32x16& G, int r, int h) {
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    float g0 = G[4 * jj], g1 = G[4 * jj + 1], g2 = G[4 * jj + 2], g3 = G[4 * jj + 3];
    if (jj == 2 && h == 0 && r == 16) g0 = 0.f;
    *reinterpret_cast<u32x2*>(&L.G16[r * GRS + 8 * jj + 4 * h]) = (u32x2){pack_f16x2(g0, g1), pack_f16x2(g2, g3)};
  }
}

// VEC: v rows 16-byte aligned with dv % 8 == 0 and out 16-byte aligned with dv % 4 == 0 (buffer
// loads and stores); otherwise element-wise accesses with bounds checks.
template <int W, bool VEC, bool OUT_F32>
__device__ __forceinline__ void output_wave(OutLds& L, const ChunkParams& p, int bh, int seg) {
  using OB = OwnedBlocks<W>;
  constexpr int NB = OB::NB;
  constexpr bool GRAM = W == kGramWave;
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  const int N = p.N, dv = p.dv;
  const size_t hrow = (size_t)bh * N;
  const uint16_t* qh = p.q + hrow * 16;
  const uint16_t* kh = p.k + hrow * 16;
  const uint16_t* vh = p.v + hrow * dv;
  const int nchunks_total = (N + CH - 1) / CH;
  const int c0 = seg * p.seg_chunks;
  const int nch = min(p.seg_chunks, nchunks_total - c0);
  constexpr int esz = OUT_F32 ? 4 : 2;

  // k-side rows of the owned slots
  int ra[NB], rb[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const KRows kr = krows(block_slot(OB::first + b, r));
    ra[b] = kr.a * KRS;
    rb[b] = kr.b * KRS;
  }
  const int grow = gram_row(r) * KRS;
  // causal mask of the diagonal score tile: element e of lane (query r, half h) is key
  // 16 (e >> 3) + 8 h + (e & 7); packed pairs keep a half iff key <= r
  u32 dmask[8];
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const int k0 = 16 * ((2 * x) >> 3) + 8 * h + ((2 * x) & 7);
    dmask[x] = (k0 <= r ? 0xffffu : 0u) | (k0 + 1 <= r ? 0xffff0000u : 0u);
  }

  // ---- state at the segment start
  f32x16 S[NB][2];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    S[b][0] = splat16(0.f);
    S[b][1] = splat16(0.f);
  }
  f32x16 G = splat16(0.f);
  StageRegs st;
  StageConv cv;
  stage_load<VEC, true>(st, p, qh, kh, vh, c0 * CH, lane, W);
  if (seg > 0) {
    const size_t slot = (size_t)bh * p.P + (seg - 1);
    const uint16_t* ws = p.wsS + slot * (64 * NF);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = OB::first + b;
#pragma unroll
      for (int n = 0; n < 2; ++n) {
#pragma unroll
        for (int J = 0; J < 2; ++J) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(&ws[(32 * n + r) * NF + 32 * blk + 16 * J + 8 * h]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            S[b][n][8 * J + 2 * i] = f16_lo_to_f32(x[i]);
            S[b][n][8 * J + 2 * i + 1] = f16_hi_to_f32(x[i]);
          }
        }
      }
    }
    if (GRAM) {
      const float* gin = p.wsG + slot * 1024 + lane * 16;
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(&gin[e]);
        G[e] = x[0];
        G[e + 1] = x[1];
        G[e + 2] = x[2];
        G[e + 3] = x[3];
      }
    }
  }

  init_kt_constants(L.KT, tid, 64 * NWAVE_OUT);
  publish_state<NB>(L, S, OB::first, r, h);
  if (GRAM) publish_gram(L, G, r, h);
  stage_convert<true>(st, cv, p.alpha, p.beta);
  stage_write<true>(cv, L.Q0, L.Q1, L.Kr, L.KT, L.VT, lane, W);
  lds_barrier();

  constexpr u32 kOnes = 0x3c003c00u;
  for (int c = 0; c < nch; ++c) {
    const int row0 = (c0 + c) * CH;
    // next chunk (unconditional, which keeps the chunk body one basic block: past the end of the
    // segment it reads the next segment's tokens or, past N, zeros, and the values go unused)
    stage_load<VEC, true>(st, p, qh, kh, vh, min(row0 + CH, N - 1), lane, W);

    // ---- phi(q) of token 32W + r (lane half h: q~ rotated by 2h elements) and the
    // inter-chunk product O^T += S^T phi(Q)^T
    u32 R[8];
    {
      const uint16_t* qrow = (h ? L.Q1 : L.Q0) + (32 * W + r) * QRS;
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(qrow);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(qrow + 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        R[i] = a0[i];
        R[4 + i] = a1[i];
      }
    }
    f32x16 O[2] = {splat16(0.f), splat16(0.f)};
#pragma unroll
    for (int kk = 0; kk < NF / 16; ++kk) {
      u32x4 bq;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const Tpl t = tpl(4 * kk + m);
        u32 v;
        if (t.t == TL) {
          v = R[t.a];
        } else if (t.t == TS) {
          v = pk_mul_f16(R[t.a], R[t.a]);
        } else if (t.t == TX) {
          v = pk_mul_f16(R[t.a], swap16(R[t.a]));
          if (t.a == 0) v = (v & 0xffffu) | 0x3c000000u;
        } else {
          v = pk_mul_f16(R[t.a], t.sw ? swap16(R[t.b]) : R[t.b]);
        }
        bq[m] = v;
      }
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&L.ST[(32 * n + r) * STS + 16 * kk + 8 * h]);
        O[n] = mfma32x32x16_f16(a, bq, O[n]);
      }
    }

    // ---- denominator of the earlier tokens: q'^T G q' with q' = [q~ | 1 | 0 ...]; T^T = G Q'^T
    // on two MFMAs, lane (token r) holds T_i for i = 8 (e >> 2) + 4 h + (e & 3)
    const u32x4 qb = *reinterpret_cast<const u32x4*>(&L.Q0[(32 * W + r) * QRS + 8 * h]);
    float dden;
    {
      const u32x4 g0 = *reinterpret_cast<const u32x4*>(&L.G16[r * GRS + 8 * h]);
      const u32x4 g1 = *reinterpret_cast<const u32x4*>(&L.G16[r * GRS + 16 + 8 * h]);
      const u32x4 one = {h == 0 ? 0x3c00u : 0u, 0u, 0u, 0u};
      f32x16 T = mfma32x32x16_f16(g0, qb, splat16(0.f));
      T = mfma32x32x16_f16(g1, one, T);
      const u32x2 qx = *reinterpret_cast<const u32x2*>(&L.Q0[(32 * W + r) * QRS + 4 * h]);
      const u32x2 qy = *reinterpret_cast<const u32x2*>(&L.Q0[(32 * W + r) * QRS + 8 + 4 * h]);
      dden = T[8];   // i = 16 + 4h: the ones component (rows past 16 of G are zero)
      dden = __builtin_fmaf(T[0], f16_lo_to_f32(qx[0]), dden);
      dden = __builtin_fmaf(T[1], f16_hi_to_f32(qx[0]), dden);
      dden = __builtin_fmaf(T[2], f16_lo_to_f32(qx[1]), dden);
      dden = __builtin_fmaf(T[3], f16_hi_to_f32(qx[1]), dden);
      dden = __builtin_fmaf(T[4], f16_lo_to_f32(qy[0]), dden);
      dden = __builtin_fmaf(T[5], f16_hi_to_f32(qy[0]), dden);
      dden = __builtin_fmaf(T[6], f16_lo_to_f32(qy[1]), dden);
      dden = __builtin_fmaf(T[7], f16_hi_to_f32(qy[1]), dden);
    }

    // ---- intra-chunk: key tiles j <= W
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j <= W; ++j) {
      const u32x4 ka = *reinterpret_cast<const u32x4*>(&L.Kr[(32 * j + perm32(r)) * QRS + 8 * h]);
      const f32x16 sc = mfma32x32x16_f16(ka, qb, splat16(1.0f));
      u32 pk[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        pk[x] = pack_f16x2(__builtin_fmaf(sc[2 * x], sc[2 * x], 1.0f), __builtin_fmaf(sc[2 * x + 1], sc[2 * x + 1], 1.0f));
        if (j == W) pk[x] &= dmask[x];
        rs = dot2_f16(pk[x], kOnes, rs);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 bp = {pk[4 * s], pk[4 * s + 1], pk[4 * s + 2], pk[4 * s + 3]};
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(&L.VT[(32 * n + r) * KRS + 32 * j + 16 * s + 8 * h]);
          O[n] = mfma32x32x16_f16(a, bp, O[n]);
        }
      }
    }

    // ---- normaliser and outputs.  Lane (token 32W + r, half h) holds dv 32n + 8jj + 4h + i
    // in O[n][4jj + i]; all values are in units of 2p.
    {
      float x = dden + rs;
      x += __shfl_xor(x, 32);
      const float den = (float)row0 + 0.5f * x;
      // v_rcp_f32 (1 ulp) instead of an IEEE division, and a select, keep this branch-free
      const float sc = p.normalize ? 0.5f * __builtin_amdgcn_rcpf(den + p.eps) : 0.5f;
      const int row = row0 + 32 * W + r;
      if (VEC) {
        const __amdgpu_buffer_rsrc_t ro =
            make_rsrc(static_cast<char*>(p.out) + ((size_t)hrow + row0) * dv * esz, (u32)(N - row0) * (u32)dv * (u32)esz);
#pragma unroll
        for (int n = 0; n < 2; ++n) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int col = 32 * n + 8 * jj + 4 * h;
            const int voff = col < dv ? ((32 * W + r) * dv + col) * esz : kOffOutOfRange;
            const float y0 = O[n][4 * jj] * sc, y1 = O[n][4 * jj + 1] * sc;
            const float y2 = O[n][4 * jj + 2] * sc, y3 = O[n][4 * jj + 3] * sc;
            if (OUT_F32)
              buf_store_b128(__builtin_bit_cast(u32x4, (f32x4){y0, y1, y2, y3}), ro, voff);
            else
              buf_store_b64((u32x2){pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)}, ro, voff);
          }
        }
      } else if (row < N) {
        const size_t obase = (size_t)(hrow + row) * dv;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int col = 32 * n + 8 * jj + 4 * h;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float y = O[n][4 * jj + i] * sc;
              if (col + i < dv) {
                if (OUT_F32)
                  static_cast<float*>(p.out)[obase + col + i] = y;
                else
                  static_cast<uint16_t*>(p.out)[obase + col + i] = f32_to_bf16_bits(y);
              }
            }
          }
        }
      }
    }

    // ---- state update with this chunk
    update_blocks<NB>(L.KT, L.VT, S, ra, rb, r, h);
    if (GRAM) gram_update(L.KT, G, grow, h, 0, 1);
    stage_convert<true>(st, cv, p.alpha, p.beta);   // next chunk, in registers
    stage_pin<true>(cv);

    lds_barrier();   // every wave is done with this chunk's tables and the published state
    if (c + 1 < nch) {
      stage_write<true>(cv, L.Q0, L.Q1, L.Kr, L.KT, L.VT, lane, W);
      publish_state<NB>(L, S, OB::first, r, h);
      if (GRAM) publish_gram(L, G, r, h);
      lds_barrier();
    }
  }

  // ---- final state of the head (last segment) in the reference feature basis, fp32:
  // state_out[f][0..dv) = sum_u phi_f(k_u) v_u, state_out[f][dv] = sum_u phi_f(k_u)
  if (p.state_out != nullptr && seg == p.P - 1) {
    float* so = p.state_out + (size_t)bh * 153 * (dv + 1);
    // the Gram matrix in fp32 for the k-sums: G32[i][j], 32 x 33 floats over the S^T table
    float* G32 = reinterpret_cast<float*>(L.ST);
    if (GRAM) {
#pragma unroll
      for (int e = 0; e < 16; ++e) G32[(8 * (e >> 2) + 4 * h + (e & 3)) * 33 + r] = G[e];
    }
    lds_barrier();
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = OB::first + b;
      // accumulator element e of lane half h is slot 32 blk + 16 (e >> 3) + 8 h + (e & 7)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int f = 32 * blk + 16 * (e >> 3) + 8 * h + (e & 7);
        const RefFeat rf = ref_feature(f);
        if (rf.ref < 0) continue;
        const float fac = p.st_fac[rf.fac];
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int col = 32 * n + r;
          if (col < dv) so[(size_t)rf.ref * (dv + 1) + col] = S[b][n][e] * fac;
        }
      }
      // k-sums of the slots of rows r of the update tile (lane half 0)
      const int f = block_slot(blk, r);
      const RefFeat rf = ref_feature(f);
      if (h == 0 && rf.ref >= 0) {
        const KRows kr = krows(f);
        int da, db;
        float fa, fb;
        kt_row_dim(kr.a, da, fa);
        kt_row_dim(kr.b, db, fb);
        const float z = fa * fb * G32[da * 33 + db];
        so[(size_t)rf.ref * (dv + 1) + dv] = rf.ref == 0 ? (float)N : z * p.st_fac[rf.fac];
      }
    }
  }
}

template <bool VEC, bool OUT_F32>
__global__ __launch_bounds__(64 * NWAVE_OUT, 2) void chunked_output_kernel(const ChunkParams p) {
  __shared__ __attribute__((aligned(16))) OutLds L;
  int bh, seg;
  map_segment(blockIdx.x, p.BH, p.P, bh, seg);
  switch (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) {
    case 0: output_wave<0, VEC, OUT_F32>(L, p, bh, seg); break;
    case 1: output_wave<1, VEC, OUT_F32>(L, p, bh, seg); break;
    case 2: output_wave<2, VEC, OUT_F32>(L, p, bh, seg); break;
    default: output_wave<3, VEC, OUT_F32>(L, p, bh, seg); break;
  }
}

// Segment split: enough (head, segment) work-groups to fill the GPU twice over, at most
// MAX_SEG segments per head.
void segment_split(int BH, int N, int& P, int& seg_chunks) {
  const int nchunks = (N + CH - 1) / CH;
  P = (512 + BH - 1) / BH;
  if (P > MAX_SEG) P = MAX_SEG;
  if (P > nchunks) P = nchunks;
  if (P < 1) P = 1;
  seg_chunks = (nchunks + P - 1) / P;
  P = (nchunks + seg_chunks - 1) / seg_chunks;
}

}  // namespace

size_t chunked_workspace_bytes(int BH, int N, int d, int dv, int chunk) {
  if (d != 16 || dv > 64 || chunk < 1) return (size_t)-1;
  int P, seg_chunks;
  segment_split(BH, N, P, seg_chunks);
  const size_t per = (size_t)64 * NF * 2 + (size_t)1024 * 4;
  return (size_t)BH * P * per + 256;
}

int launch_based_chunked(const ChunkedArgs& a, hipStream_t stream) {
  if (a.d != 16 || a.dv > 64) return LA_ERR_UNSUPPORTED_DIM;
  if (a.in_f32) return LA_ERR_BAD_DTYPE;
  if ((reinterpret_cast<uintptr_t>(a.q) & 7) || (reinterpret_cast<uintptr_t>(a.k) & 7)) return LA_ERR_BAD_ALIGNMENT;
  ChunkParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.out = a.out;
  p.state_out = a.state_out;
  p.BH = a.BH;
  p.N = a.N;
  p.dv = a.dv;
  int P, seg_chunks;
  segment_split(a.BH, a.N, P, seg_chunks);
  p.P = P;
  p.seg_chunks = seg_chunks;
  const size_t sS = (size_t)a.BH * P * 64 * NF * 2;
  char* ws = static_cast<char*>(a.workspace);
  p.wsS = reinterpret_cast<uint16_t*>(ws);
  p.wsG = reinterpret_cast<float*>(ws + sS);
  // q~ = alpha q, k~ = beta k with alpha beta = scale; sigma moves magnitude from the state
  // (sums over up to N tokens) to the q side so that it stays well inside the fp16 range.
  int sigma = 0;
  while ((1 << (sigma + 10)) < a.N && sigma < 12) sigma += 2;
  const double rc = sqrt((double)a.scale);
  p.alpha = (float)(rc * ldexp(1.0, sigma / 2));
  p.beta = (float)(rc * ldexp(1.0, -sigma / 2));
  // internal k side -> reference features: constant 2, linear 2 k~, square k~^2, pair 2 k~ k~
  p.st_fac[0] = 0.5f;
  p.st_fac[1] = (float)(ldexp(1.0, sigma / 2) * 0.5);
  p.st_fac[2] = (float)(ldexp(1.0, sigma) / sqrt(2.0));
  p.st_fac[3] = (float)(ldexp(1.0, sigma) * 0.5);
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  const bool vec_v = (a.dv % 8 == 0) && ((reinterpret_cast<uintptr_t>(a.v) & 15) == 0);
  p.vec_out = (a.dv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.out) & 15) == 0);
  if (P > 1) {
    const dim3 grid((unsigned)(a.BH * (P - 1)));
    if (vec_v)
      hipLaunchKernelGGL(chunked_segment_kernel<true>, grid, dim3(64 * NWAVE_SEG), 0, stream, p);
    else
      hipLaunchKernelGGL(chunked_segment_kernel<false>, grid, dim3(64 * NWAVE_SEG), 0, stream, p);
    int e = (int)hipGetLastError();
    if (e != 0) return e;
    const dim3 pgrid((unsigned)((64 * NF / 8 + 1024 / 4 + 255) / 256), (unsigned)a.BH);
    hipLaunchKernelGGL(chunked_prefix_kernel, pgrid, dim3(256), 0, stream, p);
    e = (int)hipGetLastError();
    if (e != 0) return e;
  }
  const dim3 grid((unsigned)(a.BH * P));
  const dim3 block(64 * NWAVE_OUT);
  const bool vec = vec_v && p.vec_out;
  if (vec && a.out_f32)
    hipLaunchKernelGGL((chunked_output_kernel<true, true>), grid, block, 0, stream, p);
  else if (vec)
    hipLaunchKernelGGL((chunked_output_kernel<true, false>), grid, block, 0, stream, p);
  else if (a.out_f32)
    hipLaunchKernelGGL((chunked_output_kernel<false, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((chunked_output_kernel<false, false>), grid, block, 0, stream, p);
  return (int)hipGetLastError();
}

}  // namespace la
