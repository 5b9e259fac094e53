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
//   * phi is never materialised in HBM.  With q~ = k~-scale = sqrt(scale) (q, k) the kernel works
//     in units of p/2:  2 p(s) = 2 + 2 s + s^2 = sum_f qf(q~) kf(k~), over 160 feature slots
//     (10 K-steps of 16) holding the 153 distinct features of the symmetric Taylor map: the
//     constant, q~_i, q~_i^2 and q~_i q~_j (i < j); the k side carries a factor 1/4, so the
//     products sum to p/2.  The q side of a K-step is four packed-fp16 products of q~'s eight
//     register pairs R_x = (q~_2x, q~_2x+1); the two lane halves of the MFMA operand hold q~
//     rotated by two registers, so one v_pk_mul_f16 yields two features for each half
//     ("templates" below).  The k side multiplies two rows of an LDS table
//     [k~/2 | 1/2 | 0 | 1] (K^T, token pairs packed), again one v_pk_mul_f16 per two products
//     (each product is 1/4 of k~_i k~_j, k~_i, 2); the factor 2 of the linear and mixed terms is
//     on the q side.
//   * Range.  fp16 (2^-14 .. 65504) carries the features, V, the state and the Gram matrix, so
//     every fp16 copy of a growing or data-sized quantity has a power-of-two exponent: V and the
//     state in registers share one exponent U per work-group (V is converted as fp16(v 2^-U) and
//     the state accumulates in units of 2^U); at every chunk boundary the waves exchange
//     max |S| and the next chunk's max |v| through LDS at the barrier they already pass, and U
//     rises (the state registers rescaled) when either would leave fp16 -- a rare event, since
//     U steps up by several binades at once.  The Gram matrix published for the denominator has
//     its own exponent; the state increments and prefixes in the workspace carry one exponent
//     per (head, segment).  Intra-chunk scores are b/2 = 1/2 + q~.k~/2 (an MFMA started from the
//     inline constant 0.5), so P/4 = (b/2)^2 + 1/4 stays in fp16 for |s| up to about 510.
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
#include <float.h>
#include <math.h>

#include "../../include/based_la.h"
#include "la_chunk_basis.hpp"
#include "la_common.hpp"
#include "la_internal.hpp"

namespace la {

namespace {

using namespace chunk_basis;

constexpr int NWAVE_OUT = 4;
constexpr int NWAVE_SEG = 5;
constexpr int MAX_SEG = 32;


// LDS image of one chunk and of the published state.
struct OutLds {
  uint16_t Q0[CH * QRS];        // q~ rows (fp16): q~_0 .. q~_15, q~_0 .. q~_3
  uint16_t Kr[CH * QRS];        // k~ rows
  uint16_t KT[KT_ROWS * KRS];   // k~^T, constant rows
  uint16_t VT[64 * KRS];        // V^T, 16-byte units swizzled by row (vt_off)
  uint16_t ST[64 * STS];        // S^T (feature slots)
  uint16_t G16[32 * GRS];       // Gram matrix of [k~/2 | 1/2] over earlier tokens in units of 2^eg, (16,16) zeroed
  u32 xs[2][NWAVE_OUT];         // per wave, by chunk parity: max |S| (fp32 bits) before the update
  u32 xv[2][NWAVE_OUT];         // max |v| (bf16 bits) of the next chunk
  u32 xk[2][NWAVE_OUT];         // max |k| (bf16 bits) of the next chunk
  int eg;                       // exponent of G16
  __attribute__((aligned(16))) u32 OS[NWAVE_OUT][32 * 32];   // per wave: its 32 output rows of a chunk (ost_off)
};
// Dword offset of 16-byte unit c (0..7) of row r in a wave's output staging rows: units are
// XOR-swizzled by r & 7, so the accumulator-order writes (ds_write_b64 / b128, lanes r = 0..15)
// and the row-order reads (ds_read_b128, eight lanes per row) hit distinct banks.
__device__ __forceinline__ int ost_off(int r, int c) { return 32 * r + 4 * (c ^ (r & 7)); }
// LDS image of the full-layer kernel: the chunk recurrence's tables with V^T in a ring of two
// chunks (slot = absolute chunk index & 1: the softmax branch reads the previous chunk's keys),
// the softmax branch's K_sw rows in a ring of two chunks, the chunk's linear-branch outputs
// (normalised, fp32) handed from the recurrence waves to the softmax waves, and the exponent of
// each V^T slot.
constexpr int YLS = 68;         // row stride (floats) of the handed-over linear outputs
template <int DSW>
struct LayerLds {
  uint16_t Q0[CH * QRS];
  uint16_t Kr[CH * QRS];
  uint16_t KT[KT_ROWS * KRS];
  uint16_t VT2[2][64 * KRS];
  uint16_t ST[64 * STS];
  uint16_t G16[32 * GRS];
  u32 xs[2][NWAVE_OUT];
  u32 xv[2][NWAVE_OUT];
  u32 xk[2][NWAVE_OUT];
  int eg;
  int Us[2];
  uint16_t KSW[2][CH * (DSW + 8)];
  float YL[CH * YLS];
};
__device__ __forceinline__ uint16_t* vtab(OutLds& L, int) { return L.VT; }
template <int DSW>
__device__ __forceinline__ uint16_t* vtab(LayerLds<DSW>& L, int slot) { return L.VT2[slot]; }

struct SegTables {
  uint16_t KT[KT_ROWS * KRS];
  uint16_t VT[64 * KRS];
};
struct SegLds {
  SegTables buf[2];
};


// ---- staging: global -> registers -> (convert) -> LDS
//
// Every load instruction of a wave reads whole 128-byte lines.  Wave wv (0..3), lane l:
//   q, k: token 32 wv + l/2, dims 8 (l % 2) .. +7 (16 B; a wave reads 1 KB contiguous);
//   v:    tokens 32 wv + 16 pp + 2 (l/8) + {0, 1} (pp = 0, 1), dims 8 (l % 8) .. +7, i.e. eight
//         full rows per instruction.
// K^T needs token pairs: lanes l and l ^ 2 hold tokens 2i, 2i + 1 and swap half their dims.
struct StageRegs {
  u32x4 q, k;
  u32x4 v[2][2];   // [pp][token of the pair]
};

// row0 < N; with valid false every load reads zero without touching memory (empty resource),
// which lets a loop issue its look-ahead load unconditionally.
template <bool VEC_V, bool WITH_Q>
__device__ __forceinline__ void stage_load(StageRegs& s, const ChunkParams& p, const uint16_t* qh,
                                           const uint16_t* kh, const uint16_t* vh, int row0, int l, int wv,
                                           bool valid = true) {
  const int N = p.N, dv = p.dv;
  const u32 rem = valid ? (u32)(N - row0) : 0u;
  {
    const int voff = (32 * wv + (l >> 1)) * 32 + 16 * (l & 1);
    s.k = buf_load_b128(make_rsrc(kh + (size_t)row0 * 16, rem * 32u), voff);
    if (WITH_Q) s.q = buf_load_b128(make_rsrc(qh + (size_t)row0 * 16, rem * 32u), voff);
  }
  const int col = 8 * (l & 7);
  if (VEC_V) {
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vh + (size_t)row0 * dv, rem * (u32)dv * 2u);
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = 32 * wv + 16 * pp + 2 * (l >> 3) + j;
        s.v[pp][j] = buf_load_b128(rv, col < dv ? (t * dv + col) * 2 : kOffOutOfRange);
      }
    }
  } else {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = row0 + 32 * wv + 16 * pp + 2 * (l >> 3) + j;
        uint16_t e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          e[i] = (valid && row < N && col + i < dv) ? vh[(size_t)row * dv + col + i] : (uint16_t)0;
        s.v[pp][j] = (u32x4){e[0] | ((u32)e[1] << 16), e[2] | ((u32)e[3] << 16), e[4] | ((u32)e[5] << 16),
                             e[6] | ((u32)e[7] << 16)};
      }
    }
  }
}

// Converted staging values of one thread: q~ / k~ row pieces (dims 8 (l % 2) .. +7), k~ token
// pairs of four dims, V^T token pairs of dims 8 (l % 8) + e for the two token pairs pp.
struct StageConv {
  u32x4 q, kr;
  u32 kt[4];
  u32 vt[2][8];
};


// q~, k~/2 pieces (stage_convert_qk) and V^T pairs as fp16(v vs) (stage_convert_v).
template <bool WITH_Q>
__device__ __forceinline__ void stage_convert_qk(const StageRegs& s, StageConv& o, float alpha, float beta, int l) {
  if (WITH_Q) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o.q[i] = pack_f16x2(alpha * bf16_lo_to_f32(s.q[i]), alpha * bf16_hi_to_f32(s.q[i]));
  }
  // K^T pairs: the even-token lane of a pair keeps dims +0..3, the odd-token lane dims +4..7
  const bool odd = (l >> 1) & 1;
  const u32 send0 = odd ? s.k[0] : s.k[2], send1 = odd ? s.k[1] : s.k[3];
  const u32 got0 = swap_quad_pairs(send0), got1 = swap_quad_pairs(send1);
  const u32 own0 = odd ? s.k[2] : s.k[0], own1 = odd ? s.k[3] : s.k[1];
  const u32 ev0 = odd ? got0 : own0, ev1 = odd ? got1 : own1;   // even token, 4 dims (bf16)
  const u32 od0 = odd ? own0 : got0, od1 = odd ? own1 : got1;   // odd token
  o.kt[0] = pack_f16x2(beta * bf16_lo_to_f32(ev0), beta * bf16_lo_to_f32(od0));
  o.kt[1] = pack_f16x2(beta * bf16_hi_to_f32(ev0), beta * bf16_hi_to_f32(od0));
  o.kt[2] = pack_f16x2(beta * bf16_lo_to_f32(ev1), beta * bf16_lo_to_f32(od1));
  o.kt[3] = pack_f16x2(beta * bf16_hi_to_f32(ev1), beta * bf16_hi_to_f32(od1));
  if (WITH_Q) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o.kr[i] = pack_f16x2(beta * bf16_lo_to_f32(s.k[i]), beta * bf16_hi_to_f32(s.k[i]));
  }
}

// The kernels' main path converts V as is (exponent 0, the usual case); when a work-group's
// exponent is not 0 a separate rare path converts it again with stage_convert_v_scaled and
// rewrites the table before the readers' barrier.  (One conversion with a run-time choice
// between the two costs registers the segment kernel does not have at three waves per SIMD.)
__device__ __forceinline__ void stage_convert_v(const StageRegs& s, StageConv& o) {
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32 a = s.v[pp][0][w], b = s.v[pp][1][w];
      o.vt[pp][2 * w] = pack_f16x2(bf16_lo_to_f32(a), bf16_lo_to_f32(b));
      o.vt[pp][2 * w + 1] = pack_f16x2(bf16_hi_to_f32(a), bf16_hi_to_f32(b));
    }
  }
}

__device__ __forceinline__ void stage_convert_v_scaled(const StageRegs& s, StageConv& o, float vs) {
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32 a = s.v[pp][0][w], b = s.v[pp][1][w];
      o.vt[pp][2 * w] = pack_f16x2(bf16_lo_to_f32(a) * vs, bf16_lo_to_f32(b) * vs);
      o.vt[pp][2 * w + 1] = pack_f16x2(bf16_hi_to_f32(a) * vs, bf16_hi_to_f32(b) * vs);
    }
  }
}

// Largest |k| of this thread's staged k values, as bf16 magnitude bits.
__device__ __forceinline__ u32 stage_kmax(const StageRegs& s) {
  typedef __attribute__((__vector_size__(2 * sizeof(unsigned short)))) unsigned short u16x2;
  u16x2 m = {0, 0};
#pragma unroll
  for (int w = 0; w < 4; ++w) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, s.k[w] & 0x7fff7fffu));
  return max((u32)m[0], (u32)m[1]);
}

// Largest |v| of this thread's staged V values, as bf16 magnitude bits.
__device__ __forceinline__ u32 stage_vmax(const StageRegs& s) {
  typedef __attribute__((__vector_size__(2 * sizeof(unsigned short)))) unsigned short u16x2;
  u16x2 m = {0, 0};
#pragma unroll
  for (int pp = 0; pp < 2; ++pp)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, s.v[pp][j][w] & 0x7fff7fffu));
  return max((u32)m[0], (u32)m[1]);
}

// Largest |x| over an accumulator array, as fp32 bits.
template <int NB>
__device__ __forceinline__ u32 acc_absmax(const f32x16 (&S)[NB][2]) {
  float m = 0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int i = 0; i < 16; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(S[b][n][i]));
  return __builtin_bit_cast(u32, m);
}

// State / V exponent after a chunk: U rises (never falls) when the state registers reach 2^14
// (new U puts them below 2^10) or the next chunk's V would reach 2^15 in units of 2^U (new U
// puts it below 2^8).  eS, eV: floor(log2) of max |S| (units of 2^U) and max |v|.
__device__ __forceinline__ int next_unit(int U, int eS, int eV) {
  int n = U;
  if (eS >= 14) n = max(n, U + eS - 9);
  if (eV - n >= 15) n = max(n, eV - 7);
  return n;
}

template <int NB>
__device__ __forceinline__ void acc_scale(f32x16 (&S)[NB][2], float f) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int i = 0; i < 16; ++i) S[b][n][i] *= f;
}

// Keeps the conversion above this point (the compiler would otherwise sink it next to the LDS
// stores, between two barriers where every wave waits for it).
template <bool WITH_Q>
__device__ __forceinline__ void stage_pin(StageConv& o) {
  if (WITH_Q) {
    asm volatile("" : "+v"(o.q[0]), "+v"(o.q[1]), "+v"(o.q[2]), "+v"(o.q[3]));
    asm volatile("" : "+v"(o.kr[0]), "+v"(o.kr[1]), "+v"(o.kr[2]), "+v"(o.kr[3]));
  }
  asm volatile("" : "+v"(o.kt[0]), "+v"(o.kt[1]), "+v"(o.kt[2]), "+v"(o.kt[3]));
#pragma unroll
  for (int pp = 0; pp < 2; ++pp)
#pragma unroll
    for (int i = 0; i < 8; i += 4) asm volatile("" : "+v"(o.vt[pp][i]), "+v"(o.vt[pp][i + 1]), "+v"(o.vt[pp][i + 2]), "+v"(o.vt[pp][i + 3]));
}

__device__ __forceinline__ void stage_write_v(const StageConv& o, uint16_t* VT, int l, int wv) {
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    const int tp = 16 * wv + 8 * pp + (l >> 3);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * (l & 7) + e;
      *reinterpret_cast<u32*>(&VT[vt_off(d, tp >> 2) + 2 * (tp & 3)]) = o.vt[pp][e];
    }
  }
}

template <bool WITH_Q>
__device__ __forceinline__ void stage_write(const StageConv& o, uint16_t* Q0, uint16_t* Kr, uint16_t* KT, uint16_t* VT,
                                            int l, int wv) {
  if (WITH_Q) {
    const int t = 32 * wv + (l >> 1), c = 8 * (l & 1);
    *reinterpret_cast<u32x4*>(&Q0[t * QRS + c]) = o.q;
    if ((l & 1) == 0) *reinterpret_cast<u32x2*>(&Q0[t * QRS + 16]) = (u32x2){o.q[0], o.q[1]};   // q~_0..3 again
    *reinterpret_cast<u32x4*>(&Kr[t * QRS + c]) = o.kr;
  }
  {
    const int tp = 16 * wv + (l >> 2);                       // token pair
    const int d0 = 8 * (l & 1) + 4 * ((l >> 1) & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32*>(&KT[kt_row(d0 + i) * KRS + 2 * tp]) = o.kt[i];
  }
  stage_write_v(o, VT, l, wv);
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
    for (int n = 0; n < 2; ++n) bv[n] = *reinterpret_cast<const u32x4*>(&VT[vt_off(32 * n + r, 2 * s + h)]);
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


// -------------------------------------------------------------------------------------------
// Kernel 1: state increment of every segment but the last.  Work-group (head, segment); wave w
// owns feature block w (all dv) and K-steps w, w + 5 of the Gram matrix; waves 0..3 stage.
// A work-group runs two segments side by side (waves 0..4 and 5..9, each with its own LDS
// tables; barriers are shared): two 5-wave work-groups per CU do not get co-scheduled, one
// 10-wave work-group spreads 3 / 3 / 2 / 2 waves over the SIMDs.
constexpr int SEG_PER_WG = 2;
template <bool VEC_V>
__global__ __launch_bounds__(64 * NWAVE_SEG * SEG_PER_WG) void chunked_segment_kernel(const ChunkParams p) {
  __shared__ __attribute__((aligned(16))) SegLds Ls[SEG_PER_WG];
  __shared__ u32 vx[2][SEG_PER_WG][4];      // max |v| of the next chunk per staging wave (by chunk parity)
  __shared__ u32 smx[SEG_PER_WG][NWAVE_SEG];   // max |S| per wave at the end
  const int wall = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = wall / NWAVE_SEG, w = wall - sub * NWAVE_SEG;
  const int tid = threadIdx.x - sub * 64 * NWAVE_SEG, lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  SegLds& L = Ls[sub];
  const int nseg_total = p.BH * (p.P - 1);
  int gseg = blockIdx.x * SEG_PER_WG + sub;
  const bool active = gseg < nseg_total;   // the last work-group may have an idle half
  if (!active) gseg = nseg_total - 1;
  int bh, seg;
  map_segment(gseg, p.BH, p.P - 1, bh, seg);
  const size_t hrow = (size_t)bh * p.N;
  const uint16_t* kh = p.k + hrow * 16;
  const uint16_t* vh = p.v + hrow * p.dv;
  const int c0 = seg * p.seg_chunks, nch = p.seg_chunks;
  const bool stager = w < 4 && active;

  const KRows kr = krows(block_slot(w, r));
  const int ra[1] = {kt_row(kr.a) * KRS}, rb[1] = {kt_row(kr.b) * KRS};
  const int grow = kt_row(gram_row(r)) * KRS;
  f32x16 S[1][2] = {{splat16(0.f), splat16(0.f)}};
  f32x16 G = splat16(0.f);

  init_kt_constants(L.buf[0].KT, tid, 64 * NWAVE_SEG);
  init_kt_constants(L.buf[1].KT, tid, 64 * NWAVE_SEG);
  // two chunks of loads in flight: chunk c + 1 sits in registers while chunk c is processed
  StageRegs sa, sb;
  StageConv cv;
  const int last = c0 + nch - 1;
  // V exponent of this half (Uo) and of the other one (Ux): every wave tracks both, so that the
  // rare extra barrier below is taken by the whole work-group; S accumulates in units of 2^Uo
  static_assert(SEG_PER_WG == 2, "two halves");
  int Uo, Ux;
  auto publish_vmax = [&](int par, const StageRegs& x, bool has) {
    const u32 m = wave_max_u32(has ? stage_vmax(x) : 0u);
    if (w < 4 && lane == 0) vx[par][sub][w] = m;
  };
  auto read_vexp = [&](int par, int sb_) -> int { return exp_of_f32bits(lds_max4(vx[par][sb_]) << 16); };
  if (stager) {
    stage_load<VEC_V, false>(sa, p, nullptr, kh, vh, c0 * CH, lane, w);
    stage_load<VEC_V, false>(sb, p, nullptr, kh, vh, min(c0 + 1, last) * CH, lane, w, nch > 1);
  }
  publish_vmax(0, sa, stager);
  if (stager) {
    stage_convert_qk<false>(sa, cv, p.qs, p.ks, lane);
    stage_convert_v(sa, cv);
    stage_write<false>(cv, nullptr, nullptr, L.buf[0].KT, L.buf[0].VT, lane, w);
  }
  lds_barrier();
  Uo = first_unit(read_vexp(0, sub));
  Ux = first_unit(read_vexp(0, sub ^ 1));
  if (Uo != 0 || Ux != 0) {   // V outside [2^-6, 2^13): convert the first chunk again, scaled
    if (Uo != 0 && stager) {
      stage_convert_v_scaled(sa, cv, __builtin_ldexpf(1.0f, -Uo));
      stage_write_v(cv, L.buf[0].VT, lane, w);
    }
    lds_barrier();
  }
  auto step = [&](int c, StageRegs& nxt, StageRegs& ahead) {
    // nxt holds chunk c + 1; ahead (free) receives chunk c + 2.  Issued by every wave (empty for
    // the non-staging one) so that the wait for nxt below counts only older loads.
    stage_load<VEC_V, false>(ahead, p, nullptr, kh, vh, min(c0 + c + 2, last) * CH, lane, w, stager && c + 2 < nch);
    const SegTables& T = L.buf[c & 1];
    // scheduling hint: interleave the state update's MFMAs with the work around them (B2 H16
    // N8192 51.74 -> 51.18 us, B1 H16 N16384 53.6 -> 53.0 us in one process, outputs identical)
    __builtin_amdgcn_iglp_opt(0);
    update_blocks<1>(T.KT, T.VT, S, ra, rb, r, h);
    gram_update(T.KT, G, grow, h, w, NWAVE_SEG);
    const bool more = stager && c + 1 < nch;
    publish_vmax((c + 1) & 1, nxt, more);
    if (more) {
      SegTables& Tn = L.buf[(c + 1) & 1];
      stage_convert_qk<false>(nxt, cv, p.qs, p.ks, lane);
      stage_convert_v(nxt, cv);
      stage_pin<false>(cv);
      stage_write<false>(cv, nullptr, nullptr, Tn.KT, Tn.VT, lane, w);
    }
    lds_barrier();
    // a half whose next V needs a higher exponent raises it and rescales its state; a half at
    // exponent != 0 converts that V again, scaled, reloading it rather than keeping its
    // registers across the barrier (uniform over the work-group)
    const int Uon = next_unit(Uo, kNoExp, read_vexp((c + 1) & 1, sub));
    const int Uxn = next_unit(Ux, kNoExp, read_vexp((c + 1) & 1, sub ^ 1));
    if (c + 1 < nch && (Uon != Uo || Uxn != Ux || Uon != 0 || Uxn != 0)) {
      if (Uon != Uo) acc_scale<1>(S, __builtin_ldexpf(1.0f, Uo - Uon));
      if (Uon != 0 && more) {
        StageRegs again;
        stage_load<VEC_V, false>(again, p, nullptr, kh, vh, (c0 + c + 1) * CH, lane, w);
        stage_convert_v_scaled(again, cv, __builtin_ldexpf(1.0f, -Uon));
        stage_write_v(cv, L.buf[(c + 1) & 1].VT, lane, w);
      }
      Uo = Uon;
      Ux = Uxn;
      lds_barrier();
    }
  };
  for (int c = 0; c < nch; c += 2) {
    step(c, sb, sa);
    if (c + 1 < nch) step(c + 1, sa, sb);
  }
  // increment: S^T fp16 [dv][slot] in units of 2^EI, EI from max |S| over the waves (values
  // below 2^14); Gram partials of the waves summed through LDS
  const size_t slot = (size_t)bh * p.P + seg;
  uint16_t* ws = p.wsS + slot * (64 * NF);
  {
    const u32 m = wave_max_u32(acc_absmax<1>(S));
    if (lane == 0) smx[sub][w] = m;
  }
  float* red = reinterpret_cast<float*>(&L);   // 5 x 64 x 16 floats = 20 KB, tables no longer read
#pragma unroll
  for (int e = 0; e < 16; e += 4)
    *reinterpret_cast<f32x4*>(&red[(w * 64 + lane) * 16 + e]) = (f32x4){G[e], G[e + 1], G[e + 2], G[e + 3]};
  lds_barrier();
  u32 msub = 0u;
#pragma unroll
  for (int i = 0; i < NWAVE_SEG; ++i) msub = max(msub, smx[sub][i]);
  msub = (u32)__builtin_amdgcn_readfirstlane((int)msub);
  const int eS = exp_of_f32bits(msub);
  // S 2^es in fp16, es = 13 - eS, clamped so that the factor stays finite (the stored exponent
  // follows the clamp; a state more than 2^114 below 1 in units of 2^Uo has lost nothing of use)
  const int es = eS == kNoExp ? 0 : min(13 - eS, 127);
  const int EI = eS == kNoExp ? kNoExp : Uo - es;
  const float f = eS == kNoExp ? 0.f : __builtin_ldexpf(1.0f, es);
#pragma unroll
  for (int n = 0; n < (active ? 2 : 0); ++n) {
#pragma unroll
    for (int J = 0; J < 2; ++J) {
      const f32x16& a = S[0][n];
      const u32x4 pk = {pack_f16x2(a[8 * J + 0] * f, a[8 * J + 1] * f), pack_f16x2(a[8 * J + 2] * f, a[8 * J + 3] * f),
                        pack_f16x2(a[8 * J + 4] * f, a[8 * J + 5] * f), pack_f16x2(a[8 * J + 6] * f, a[8 * J + 7] * f)};
      *reinterpret_cast<u32x4*>(&ws[(32 * n + r) * NF + 32 * w + 16 * J + 8 * h]) = pk;
    }
  }
  if (w == 0 && lane == 0 && active) p.wsE[slot] = EI;
  if (w == 0 && active) {
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
// Initial state (continuation): the caller's [S | z] in the reference feature basis
// (benchmarks/chunked_attention_benchmark.py:34-53 order), converted to the internal basis in
// slot P - 1 of every head: S^T slot f = S_ref[ref(f)] / (4 factor) (fp16 [64][NF] in units of
// 2^wsE, wsE from the largest entry); the Gram matrix of [k~/2 | 1/2] in the accumulator layout
// [64 lanes][16], entry (i, j) = the k-sum of the feature it carries / (4 factor): (16, 16) the
// count, (i, 16) linear, (i, i) square, (i, j) pair -- the inverse of the state export at the
// end of output_wave.
__global__ __launch_bounds__(256) void chunked_import_kernel(const ChunkParams p) {
  __shared__ u32 wm[4];
  const int bh = blockIdx.x, tid = threadIdx.x, dv = p.dv;
  const float* si = p.state_in + (size_t)bh * 153 * (dv + 1);
  const size_t slot = (size_t)bh * p.P + (p.P - 1);
  uint16_t* ws = p.wsS + slot * (64 * NF);
  auto value = [&](int idx) -> float {
    const int c = idx / NF, f = idx - c * NF;
    float x = 0.f;
    if (c < dv && f < 160) {
      const RefFeat rf = ref_feature(f);
      if (rf.ref >= 0) x = si[(size_t)rf.ref * (dv + 1) + c] * (0.25f * p.st_inv[rf.fac]);
    }
    return x;
  };
  float m = 0.f;
  for (int idx = tid; idx < 64 * NF; idx += 256) m = __builtin_fmaxf(m, __builtin_fabsf(value(idx)));
  const u32 mw = wave_max_u32(__builtin_bit_cast(u32, m));
  if ((tid & 63) == 0) wm[tid >> 6] = mw;
  __syncthreads();
  const int eS = exp_of_f32bits(max(max(wm[0], wm[1]), max(wm[2], wm[3])));
  // the caller's state at any magnitude: the power of two by ldexp on each value (exact and finite)
  const int es = eS == kNoExp ? 0 : 13 - eS;
  if (tid == 0) p.wsE[slot] = eS == kNoExp ? kNoExp : eS - 13;
  for (int idx = tid; idx < 64 * NF; idx += 256)
    ws[idx] = (uint16_t)(pack_f16x2(__builtin_ldexpf(value(idx), es), 0.f) & 0xffffu);
  float* g = p.wsG + slot * 1024;
  for (int idx = tid; idx < 1024; idx += 256) {
    const int lane = idx >> 4, e = idx & 15, r = lane & 31, h = lane >> 5;
    const int row = 8 * (e >> 2) + 4 * h + (e & 3), col = r;
    float x = 0.f;
    if (row <= 16 && col <= 16) {
      const int lo = row < col ? row : col, hi = row < col ? col : row;
      if (lo == 16) {
        x = si[dv];                                                               // count
      } else if (hi == 16) {
        x = si[(size_t)(1 + lo) * (dv + 1) + dv] * p.st_inv[1];                  // linear
      } else if (lo == hi) {
        x = si[(size_t)(17 + lo) * (dv + 1) + dv] * p.st_inv[2];                 // square
      } else {
        x = si[(size_t)(33 + lo * (31 - lo) / 2 + (hi - lo - 1)) * (dv + 1) + dv] * p.st_inv[3];   // pair
      }
    }
    g[idx] = 0.25f * x;
  }
}

// -------------------------------------------------------------------------------------------
// Kernel 2: exclusive prefixes over segments, in place: afterwards slot p - 1 holds the sum of
// the increments of segments 0 .. p-1.  Thread (head, 8-byte unit), fp32 accumulation, the loads
// of up to 16 segments in flight at once.
// With an initial state the scan starts from slot P - 1 (written by chunked_import_kernel).
// Exponents: increment s is fp16 in units of 2^wsE[s] (entries below 2^14); the prefix through
// s, a sum of n such increments, is stored in units of 2^wsEP[s] with wsEP[s] = max wsE +
// ceil(log2 n), which keeps it below 2^14 whatever the signs (the same for every thread, so
// thread 0 of the head's first work-group writes it).
__global__ __launch_bounds__(256) void chunked_prefix_kernel(const ChunkParams p) {
  constexpr int US = 64 * NF / 4, UG = 1024 / 2;   // 8-byte units of S^T (fp16) and G (fp32)
  const int e = blockIdx.x * 256 + threadIdx.x, bh = blockIdx.y;
  const int nseg = p.P - 1;
  const bool init = p.state_in != nullptr;
  if (e < US) {
    uint16_t* base = p.wsS + (size_t)bh * p.P * (64 * NF) + 4 * (size_t)e;
    // the head's exponents, read once into scalar registers (uniform addresses); fully unrolled
    // over MAX_SEG so that every index is a constant
    const int* exg = p.wsE + (size_t)bh * p.P;
    int ex[MAX_SEG];
#pragma unroll
    for (int i = 0; i < MAX_SEG; ++i) ex[i] = i < p.P ? __builtin_amdgcn_readfirstlane(exg[i]) : kNoExp;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int emax = kNoExp, cnt = 0;
    if (init) {
      const u32x2 x0 = *reinterpret_cast<const u32x2*>(base + (size_t)nseg * (64 * NF));
      emax = exg[nseg];
      cnt = 1;
      acc[0] = __builtin_ldexpf(f16_lo_to_f32(x0[0]), emax);
      acc[1] = __builtin_ldexpf(f16_hi_to_f32(x0[0]), emax);
      acc[2] = __builtin_ldexpf(f16_lo_to_f32(x0[1]), emax);
      acc[3] = __builtin_ldexpf(f16_hi_to_f32(x0[1]), emax);
    }
#pragma unroll
    for (int s0 = 0; s0 < MAX_SEG; s0 += 16) {
      if (s0 >= nseg) break;
      u32x2 x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        x[i] = s0 + i < nseg ? *reinterpret_cast<const u32x2*>(base + (size_t)(s0 + i) * (64 * NF)) : (u32x2){0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (s0 + i >= nseg) break;
        const int es = ex[s0 + i];
        emax = max(emax, es);
        ++cnt;
        const int ep = emax == kNoExp ? kNoExp : emax + (cnt > 1 ? 32 - __builtin_clz((unsigned)(cnt - 1)) : 0);
        // powers of two by ldexp on each value: exact, and finite at any exponent (an increment
        // or prefix with exponent kNoExp is all zeros, which ldexp keeps zero)
        acc[0] += __builtin_ldexpf(f16_lo_to_f32(x[i][0]), es);
        acc[1] += __builtin_ldexpf(f16_hi_to_f32(x[i][0]), es);
        acc[2] += __builtin_ldexpf(f16_lo_to_f32(x[i][1]), es);
        acc[3] += __builtin_ldexpf(f16_hi_to_f32(x[i][1]), es);
        *reinterpret_cast<u32x2*>(base + (size_t)(s0 + i) * (64 * NF)) =
            (u32x2){pack_f16x2(__builtin_ldexpf(acc[0], -ep), __builtin_ldexpf(acc[1], -ep)),
                    pack_f16x2(__builtin_ldexpf(acc[2], -ep), __builtin_ldexpf(acc[3], -ep))};
        if (e == 0) p.wsEP[(size_t)bh * p.P + s0 + i] = ep;
      }
    }
  } else if (e < US + UG) {
    float* base = p.wsG + (size_t)bh * p.P * 1024 + 2 * (size_t)(e - US);
    f32x2 acc = init ? *reinterpret_cast<const f32x2*>(base + (size_t)nseg * 1024) : (f32x2){0.f, 0.f};
    for (int s0 = 0; s0 < nseg; s0 += 16) {
      f32x2 x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        x[i] = s0 + i < nseg ? *reinterpret_cast<const f32x2*>(base + (size_t)(s0 + i) * 1024) : (f32x2){0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (s0 + i >= nseg) break;
        acc += x[i];
        *reinterpret_cast<f32x2*>(base + (size_t)(s0 + i) * 1024) = acc;
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

template <int NB, class LT>
__device__ __forceinline__ void publish_state(LT& L, const f32x16 (&S)[NB][2], int first, int r, int h) {
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
// exactly), in units of 2^eg with eg from its largest entry (entries below 2^14).  Lane (col
// j = r, rows 8 jj + 4 h + i) writes row j by symmetry.
template <class LT>
__device__ __forceinline__ void publish_gram(LT& L, const f32x16& G, int r, int h) {
  float g[16];
  float m = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    g[e] = (e == 8 && h == 0 && r == 16) ? 0.f : G[e];
    m = __builtin_fmaxf(m, __builtin_fabsf(g[e]));
  }
  const int eg0 = exp_of_f32bits(wave_max_u32(__builtin_bit_cast(u32, m)));
  const int eg = eg0 == kNoExp ? 0 : eg0 - 13;
  const float f = __builtin_ldexpf(1.0f, -eg);
#pragma unroll
  for (int jj = 0; jj < 4; ++jj)
    *reinterpret_cast<u32x2*>(&L.G16[r * GRS + 8 * jj + 4 * h]) =
        (u32x2){pack_f16x2(g[4 * jj] * f, g[4 * jj + 1] * f), pack_f16x2(g[4 * jj + 2] * f, g[4 * jj + 3] * f)};
  if (r == 0 && h == 0) L.eg = eg;
}

// Softmax branch of the full layer for one wave: queries 32W .. 32W + 31 of every chunk of the
// segment, keys t - window + 1 .. t (window <= 64), scores on bf16 MFMAs over DSW dims, online
// softmax in fp32 (exp2 of log2-scaled scores), P in fp16 against the recurrence's fp16 V^T
// (units 2^U), the outputs added to the recurrence's handed-over ones and stored
// (benchmarks/sliding_attention_benchmark.py:32-56 for the branch, kernels/nki_attention_sliding.py:4-5
// for the sum).  K_sw rows of the chunk are staged by the four softmax waves, a 32-row quarter each;
// those of the 64 tokens before the segment, and their V, in the prologue.
template <int DSW>
struct SwRole {
  static constexpr int KS = DSW > 0 ? DSW / 16 : 1;   // K-steps of a score tile; 16-byte pieces per lane
  static constexpr int KSS = DSW + 8;                  // K_sw row stride (halves)
  u32x4 qf[KS];          // Q_sw of the chunk's queries: lane (query r, half h) holds dims 16 kk + 8 h ..
  u32x4 kst[KS];         // the next chunk's K_sw quarter, in flight
  f32x16 O[2];           // numerator of the branch, V^T units of the chunk
  float ysc;             // 2^U / (softmax row sum)
  __amdgpu_buffer_rsrc_t rq, rk;
  size_t hrow;

  __device__ __forceinline__ void init(const ChunkParams& p, int bh, int, int) {
    hrow = (size_t)bh * p.N;
    rq = make_rsrc(p.qsw + hrow * DSW, (u32)p.N * (u32)(DSW * 2));
    rk = make_rsrc(p.ksw + hrow * DSW, (u32)p.N * (u32)(DSW * 2));
  }
  __device__ __forceinline__ void load_k(int cabs, int W, int lane) {
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int pc = lane + 64 * i, row = pc / (DSW / 8), c8 = pc % (DSW / 8);
      kst[i] = buf_load_b128(rk, ((cabs * CH + 32 * W + row) * DSW + 8 * c8) * 2);
    }
  }
  template <class LT>
  __device__ __forceinline__ void store_k(LT& L, int cabs, int W, int lane) {
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int pc = lane + 64 * i, row = pc / (DSW / 8), c8 = pc % (DSW / 8);
      *reinterpret_cast<u32x4*>(&L.KSW[cabs & 1][(32 * W + row) * KSS + 8 * c8]) = kst[i];
    }
  }
  __device__ __forceinline__ void load_q(int cabs, int W, int lane) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qf[kk] = buf_load_b128(rq, ((cabs * CH + 32 * W + r) * DSW + 16 * kk + 8 * h) * 2);
  }
  // V of this wave's 16 of the 64 tokens before chunk c0 (zero before the sequence) into columns
  // 64 + 16 W .. of the previous chunk's V^T slot, as fp16(v 2^-U); lane = V^T row (dv column)
  template <class LT>
  __device__ __forceinline__ void prev_v(LT& L, const ChunkParams& p, int c0, int U, int W, int lane) {
    const uint16_t* vh = p.v + hrow * p.dv;
    const float vs = __builtin_ldexpf(1.0f, -U);
    uint16_t* vt = vtab(L, (c0 + 1) & 1);
#pragma unroll
    for (int tp = 0; tp < 8; ++tp) {
      const int col = 64 + 16 * W + 2 * tp;          // chunk-local column of the previous chunk
      const int t = c0 * CH - CH + col;               // its token
      float a = 0.f, b = 0.f;
      if (lane < p.dv && t >= 0) {
        a = bf16_lo_to_f32(vh[(size_t)t * p.dv + lane]) * vs;
        b = bf16_lo_to_f32(vh[(size_t)(t + 1) * p.dv + lane]) * vs;
      }
      *reinterpret_cast<u32*>(&vt[vt_off(lane, col >> 3) + (col & 7)]) = pack_f16x2(a, b);
    }
    if (W == 0 && lane == 0) L.Us[(c0 + 1) & 1] = U;
  }
  template <class LT>
  __device__ __forceinline__ void prologue(LT& L, const ChunkParams& p, int c0, int U, int W, int lane) {
    load_k(c0, W, lane);
    load_q(c0, W, lane);
    // K_sw rows of this wave's 16 of the 64 tokens before chunk c0
    for (int pc = lane; pc < 16 * (DSW / 8); pc += 64) {
      const int row = pc / (DSW / 8), c8 = pc % (DSW / 8);
      const int t = c0 * CH - 64 + 16 * W + row;
      const u32x4 x = buf_load_b128(rk, t >= 0 ? (t * DSW + 8 * c8) * 2 : kOffOutOfRange);
      *reinterpret_cast<u32x4*>(&L.KSW[(c0 + 1) & 1][(64 + 16 * W + row) * KSS + 8 * c8]) = x;
    }
    prev_v(L, p, c0, U, W, lane);
    store_k(L, c0, W, lane);
  }
  template <class LT>
  __device__ __forceinline__ void phase1(LT& L, const ChunkParams& p, int cabs, int W, int lane, bool more) {
    if (more) load_k(cabs + 1, W, lane);
    const int r = lane & 31, h = lane >> 5, qs = 32 * W, q = qs + r;
    const int Uc = __builtin_amdgcn_readfirstlane(L.Us[cabs & 1]);
    const int Upv = __builtin_amdgcn_readfirstlane(L.Us[(cabs + 1) & 1]);
    O[0] = splat16(0.f);
    O[1] = splat16(0.f);
    float mrun = -FLT_MAX, lrun = 0.f;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int kb = qs - 64 + 32 * j;                       // chunk-local first key of the tile
      if (kb + 31 < qs - p.window + 1 || cabs * CH + kb + 31 < 0) continue;   // outside every window
      const bool prev = kb < 0;
      const int slot = prev ? (cabs + 1) & 1 : cabs & 1;
      const int kc = prev ? kb + CH : kb;
      // S^T = K_sw Q_sw^T with the key rows in perm32 order: the accumulator is the P.V operand
      f32x16 sc = splat16(0.f);
      const uint16_t* krow = &L.KSW[slot][(kc + perm32(r)) * KSS + 8 * h];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) sc = mfma32x32x16(*reinterpret_cast<const u32x4*>(krow + 16 * kk), qf[kk], sc);
      // element e of lane (query r, half h) is key kb + 16 (e >> 3) + 8 h + (e & 7)
      float x[16];
      float mt = -FLT_MAX;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kb + 16 * (e >> 3) + 8 * h + (e & 7);
        const bool ok = key <= q && key > q - p.window && cabs * CH + key >= 0;
        x[e] = ok ? sc[e] * p.sw_log2 : -FLT_MAX;
        mt = __builtin_fmaxf(mt, x[e]);
      }
      mt = __builtin_fmaxf(mt, __shfl_xor(mt, 32));   // both halves of the query's row
      const float mnew = __builtin_fmaxf(mrun, mt);
      const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
      lrun *= alpha;
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int e = 0; e < 16; ++e) O[n][e] *= alpha;
      mrun = mnew;
      // previous chunk's V^T in its own units: P scaled by 2^(U_prev - U) (1 unless U rose)
      const float pf = prev ? __builtin_ldexpf(1.0f, Upv - Uc) : 1.0f;
      u32 pk[8];
#pragma unroll
      for (int xx = 0; xx < 8; ++xx) {
        const float p0 = x[2 * xx] == -FLT_MAX ? 0.f : __builtin_amdgcn_exp2f(x[2 * xx] - mnew);
        const float p1 = x[2 * xx + 1] == -FLT_MAX ? 0.f : __builtin_amdgcn_exp2f(x[2 * xx + 1] - mnew);
        lrun += p0 + p1;
        pk[xx] = pack_f16x2(p0 * pf, p1 * pf);
      }
      const uint16_t* vt = vtab(L, slot);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 bp = {pk[4 * s], pk[4 * s + 1], pk[4 * s + 2], pk[4 * s + 3]};
#pragma unroll
        for (int n = 0; n < 2; ++n)
          O[n] = mfma32x32x16_f16(*reinterpret_cast<const u32x4*>(&vt[vt_off(32 * n + r, kc / 8 + 2 * s + h)]), bp, O[n]);
      }
    }
    const float l = lrun + __shfl_xor(lrun, 32);   // > 0: each query's own key is in its window
    ysc = __builtin_ldexpf(1.0f, Uc) / l;
  }
  template <bool OUT_F32, class LT>
  __device__ __forceinline__ void phase2(LT& L, const ChunkParams& p, int cabs, int W, int lane, bool more) {
    constexpr int esz = OUT_F32 ? 4 : 2;
    const int r = lane & 31, h = lane >> 5, qs = 32 * W, row0 = cabs * CH, dv = p.dv;
    const __amdgpu_buffer_rsrc_t ro =
        make_rsrc(static_cast<char*>(p.out) + (hrow + row0) * dv * esz, (u32)(p.N - row0) * (u32)dv * (u32)esz);
#pragma unroll
    for (int n = 0; n < 2; ++n) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int col = 32 * n + 8 * jj + 4 * h;
        const f32x4 yl = *reinterpret_cast<const f32x4*>(&L.YL[(qs + r) * YLS + col]);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = yl[e] + O[n][4 * jj + e] * ysc;
        const int voff = col < dv ? ((qs + r) * dv + col) * esz : kOffOutOfRange;
        if (OUT_F32)
          buf_store_b128(__builtin_bit_cast(u32x4, (f32x4){y[0], y[1], y[2], y[3]}), ro, voff);
        else
          buf_store_b64((u32x2){pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])}, ro, voff);
      }
    }
    if (more) {
      store_k(L, cabs + 1, W, lane);
      load_q(cabs + 1, W, lane);
    }
  }
};

// VEC: v rows 16-byte aligned with dv % 8 == 0 and out 16-byte aligned with dv % 4 == 0 (buffer
// loads and stores); otherwise element-wise accesses with bounds checks.
//
// Units: the state registers S hold (sum phi_k v) / 4 in units of 2^U (the k-side table carries
// the 1/4), the published S^T is fp16(S), V^T is fp16(v 2^-U), the intra-chunk P is fp16(p / 2),
// so O = S^T phi(Q)^T + V^T P^T is num / 2 in units of 2^U.  The Gram registers G hold
// (sum g g^T) / 4 and the published copy G16 is fp16(G 2^-EG).
//
// Full layer (LT = LayerLds<DSW>, DSW > 0): the work-group has 8 waves.  ROLE 0..3 run the chunk
// recurrence as above but hand their normalised outputs to LDS; ROLE 4..7 compute the
// sliding-window softmax of the same 32 queries (window <= 64: key tiles 64 and 32 tokens before
// the queries and their own, from the V^T ring and the K_sw ring), add the handed-over linear
// outputs and store.  Every barrier sits in code both roles run, with uniform conditions, so the
// roles pass the same barriers.
template <int ROLE, bool VEC, bool OUT_F32, class LT = OutLds, int DSW = 0>
__device__ __forceinline__ void output_wave(LT& L, const ChunkParams& p, int bh, int seg) {
  constexpr bool LAYER = DSW > 0;
  constexpr bool LIN = ROLE < NWAVE_OUT;   // recurrence role (the only one without LAYER)
  constexpr int W = LIN ? ROLE : ROLE - NWAVE_OUT;
  static_assert(!LAYER || VEC, "the layer kernel takes the vector path");
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
  const int c0 = seg * p.ostride * p.seg_chunks;
  const int nch = min(p.ostride * p.seg_chunks, nchunks_total - c0);
  constexpr int esz = OUT_F32 ? 4 : 2;

  // k-side rows of the owned slots
  int ra[NB], rb[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const KRows kr = krows(block_slot(OB::first + b, r));
    ra[b] = kt_row(kr.a) * KRS;
    rb[b] = kt_row(kr.b) * KRS;
  }
  const int grow = kt_row(gram_row(r)) * KRS;
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
  int U = kNoExp;   // exponent of the state registers and of V^T (the same in every wave)
  StageRegs st;
  StageConv cv;
  if constexpr (LIN) stage_load<VEC, true>(st, p, qh, kh, vh, c0 * CH, lane, W);
  if (seg > 0 || p.state_in != nullptr) {
    // prefix of the earlier segments (with the caller's initial state, when there is one); the
    // first segment's is slot P - 1, which holds the initial state alone
    const size_t slot = (size_t)bh * p.P + (seg > 0 ? seg * p.ostride - 1 : p.P - 1);
    U = seg > 0 ? p.wsEP[slot] : p.wsE[slot];
    const uint16_t* ws = p.wsS + slot * (64 * NF);
#pragma unroll
    for (int b = 0; b < (LIN ? NB : 0); ++b) {
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
    if (GRAM && LIN) {
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

  // Exponent of the first chunk: at least the prefix's, else first_unit of the chunk's max |v|.
  // The tables are written with a guess (the prefix's exponent, at least 0), which is right
  // unless that V lies outside [2^-6, 2^13) or the prefix's exponent is negative; then they are
  // written again behind one more barrier (the same decision in every wave).
  const int Up = U;   // kNoExp without a prefix
  U = max(Up, 0);
  // softmax role: its slice of the sliding-window branch (queries 32W .. 32W + 31 of each chunk)
  SwRole<DSW> sw;
  if constexpr (LIN) {
    if (Up != kNoExp && U != Up) acc_scale<NB>(S, __builtin_ldexpf(1.0f, Up - U));
    init_kt_constants(L.KT, tid, 64 * NWAVE_OUT);
    publish_state<NB>(L, S, OB::first, r, h);
    if (GRAM) publish_gram(L, G, r, h);
    stage_convert_qk<true>(st, cv, p.qs, p.ks, lane);
    if (U == 0)
      stage_convert_v(st, cv);
    else
      stage_convert_v_scaled(st, cv, __builtin_ldexpf(1.0f, -U));
    stage_write<true>(cv, L.Q0, L.Kr, L.KT, vtab(L, c0 & 1), lane, W);
    {
      const u32 mvk = wave_max_u16x2((stage_vmax(st) << 16) | stage_kmax(st));
      if (lane == 0) {
        L.xv[0][W] = mvk >> 16;
        L.xk[0][W] = mvk & 0xffffu;
      }
    }
    if constexpr (LAYER) {
      if (W == 0 && lane == 0) L.Us[c0 & 1] = U;
    }
  } else {
    sw.init(p, bh, W, lane);
    sw.prologue(L, p, c0, U, W, lane);
  }
  lds_barrier();
  // the current chunk's max |v| and |k| exponents, for the bound on its state increment
  int eVc = exp_of_f32bits(lds_max4(L.xv[0]) << 16);
  int eKc = exp_of_f32bits(lds_max4(L.xk[0]) << 16);
  {
    const int U0 = max(Up, first_unit(eVc));
    if (U0 != U) {   // rare, and the same in every wave (both roles)
      if constexpr (LIN) {
        acc_scale<NB>(S, __builtin_ldexpf(1.0f, U - U0));
        publish_state<NB>(L, S, OB::first, r, h);
        stage_convert_v_scaled(st, cv, __builtin_ldexpf(1.0f, -U0));
        stage_write_v(cv, vtab(L, c0 & 1), lane, W);
        if constexpr (LAYER) {
          if (W == 0 && lane == 0) L.Us[c0 & 1] = U0;
        }
      } else {
        sw.prev_v(L, p, c0, U0, W, lane);   // the previous 64 tokens' V again, with U0
      }
      U = U0;
      lds_barrier();
    }
  }

  constexpr u32 kOnes = 0x3c003c00u;
  for (int c = 0; c < nch; ++c) {
    // Two work-groups share a CU and the older one's waves issue first at equal priority, so
    // the younger one fell behind and ended alone.  Waves at an even chunk take priority 1, at
    // an odd one 0: of two work-groups a chunk apart the one at the even chunk issues first,
    // which alternates between them and keeps their progress within about a chunk (B1 H16
    // N65536 157.0 -> 153.1 us, B2 H16 N4096 40.7 -> 40.2 us in one process, outputs identical).
    if (c & 1)
      __builtin_amdgcn_s_setprio(0);
    else
      __builtin_amdgcn_s_setprio(1);
    const int row0 = (c0 + c) * CH;
    const bool more = c + 1 < nch;
    if constexpr (!LIN) {
      sw.phase1(L, p, c0 + c, W, lane, more);
      lds_barrier();   // the recurrence waves' barrier after their chunk (same position)
      sw.template phase2<OUT_F32>(L, p, c0 + c, W, lane, more);
      if (more) lds_barrier();
      continue;
    }
    // max |S| of the state this chunk starts from (its MFMAs have completed: it was published)
    const u32 msS = wave_max_u32(acc_absmax<NB>(S));
    // next chunk, issued unconditionally (one basic block); after the last chunk it reads nothing
    stage_load<VEC, true>(st, p, qh, kh, vh, min(row0 + CH, N - 1), lane, W, c + 1 < nch);

    // ---- phi(q) of token 32W + r (lane half h: q~ rotated by 2h elements) and the
    // inter-chunk product O^T += S^T phi(Q)^T
    u32 R[8], R2[8];
    {
      // elements 4h .. 4h + 15 of the extended row: q~ rotated by 2h register pairs
      const uint16_t* qrow = L.Q0 + (32 * W + r) * QRS + 4 * h;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x2 a = *reinterpret_cast<const u32x2*>(qrow + 4 * i);
        R[2 * i] = a[0];
        R[2 * i + 1] = a[1];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) R2[i] = pk_mul_f16(R[i], 0x40004000u);
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
          v = R2[t.a];
        } else if (t.t == TS) {
          v = pk_mul_f16(R[t.a], R[t.a]);
        } else if (t.t == TX) {
          v = pk_mul_f16(R2[t.a], swap16(R[t.a]));
          if (t.a == 0) v = (v & 0xffffu) | 0x3c000000u;
        } else {
          v = pk_mul_f16(R2[t.a], t.sw ? swap16(R[t.b]) : R[t.b]);
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
      dden *= __builtin_ldexpf(1.0f, __builtin_amdgcn_readfirstlane(L.eg));
    }

    // ---- intra-chunk: key tiles j <= W; scores b/2 = 1/2 + q~.(k~/2), P = (b/2)^2 + 1/4 = p/2.
    // The call's first 64 queries (waves 0 and 1 of its first chunk) also take P's fp16 remainder
    // lo = fp16(P - fp16(P)) through a second P.V MFMA: without an initial state these rows'
    // outputs average a few tokens' v, far above the head's rms (what the parity metric divides
    // by), and hi + lo keeps ~22 bits of P; later rows average enough keys that fp16 P alone is
    // well inside the bar (worst head of B2 H16 N8192: 2.1e-2 without these rows, 3.7e-3 with
    // them; of B1 H16 N65536: 8.7e-3 with them).
    // Taken with an initial state too, so that a zero state gives the plain call's result; only
    // in waves 0 and 1 of the vector-path kernels, whose loops carry the extra code without
    // spilling or slowing down.
    const bool exact = W <= 1 && VEC && !LAYER && row0 == 0;
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j <= W; ++j) {
      const u32x4 ka = *reinterpret_cast<const u32x4*>(&L.Kr[(32 * j + perm32(r)) * QRS + 8 * h]);
      const f32x16 sc = mfma32x32x16_f16(ka, qb, splat16(0.5f));
      u32 pk[8], pl[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        pk[x] = sq_plus_f16x2(sc[2 * x], sc[2 * x + 1], 0.25f);
        if (exact) {
          const float pa = __builtin_fmaf(sc[2 * x], sc[2 * x], 0.25f), pb = __builtin_fmaf(sc[2 * x + 1], sc[2 * x + 1], 0.25f);
          pl[x] = pack_f16x2(pa - f16_lo_to_f32(pk[x]), pb - f16_hi_to_f32(pk[x]));
        } else {
          pl[x] = 0u;
        }
        if (j == W) {
          pk[x] &= dmask[x];
          pl[x] &= dmask[x];
        }
        rs = dot2_f16(pk[x], kOnes, rs);
        if (exact) rs = dot2_f16(pl[x], kOnes, rs);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 bp = {pk[4 * s], pk[4 * s + 1], pk[4 * s + 2], pk[4 * s + 3]};
        const u32x4 bl = {pl[4 * s], pl[4 * s + 1], pl[4 * s + 2], pl[4 * s + 3]};
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(&vtab(L, (c0 + c) & 1)[vt_off(32 * n + r, 4 * j + 2 * s + h)]);
          O[n] = mfma32x32x16_f16(a, bp, O[n]);
          if (exact) O[n] = mfma32x32x16_f16(a, bl, O[n]);
        }
      }
    }

    // ---- normaliser and outputs.  Lane (token 32W + r, half h) holds dv 32n + 8jj + 4h + i
    // in O[n][4jj + i]; O is num / 2 in units of 2^U, dden and rs are sums of p/2 - 1/2 and p/2.
    {
      float x = dden + rs;
      x += __shfl_xor(x, 32);
      const float den = (float)row0 + p.prev_tokens + 2.0f * x;
      const float un = __builtin_ldexpf(2.0f, U);
      // v_rcp_f32 (1 ulp) instead of an IEEE division, and a select, keep this branch-free
      const float sc = p.normalize ? un * __builtin_amdgcn_rcpf(den + p.eps) : un;
      const int row = row0 + 32 * W + r;
      if (!LAYER && p.den_out != nullptr && h == 0 && row < N) p.den_out[(size_t)hrow + row] = den;
      if constexpr (LAYER) {
        // handed to the softmax wave of these queries, which adds its branch and stores
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            *reinterpret_cast<f32x4*>(&L.YL[(32 * W + r) * YLS + 32 * n + 8 * jj + 4 * h]) =
                (f32x4){O[n][4 * jj] * sc, O[n][4 * jj + 1] * sc, O[n][4 * jj + 2] * sc, O[n][4 * jj + 3] * sc};
      } else if (VEC) {
        // The wave's 32 x dv tile goes through its staging rows in LDS, so that every store
        // instruction writes eight whole 128-byte row pieces (lane: row 8 i + l / 8, unit l % 8)
        // instead of 16-byte pieces of 32 rows.  bf16: one pass of 64 columns; fp32: one pass per
        // 32-column half.  Only this wave touches its rows (LDS operations of a wave complete in
        // order).
        const __amdgpu_buffer_rsrc_t ro =
            make_rsrc(static_cast<char*>(p.out) + ((size_t)hrow + row0) * dv * esz, (u32)(N - row0) * (u32)dv * (u32)esz);
        u32* os = L.OS[W];
        const int rr = lane >> 3, cu = lane & 7;
        if constexpr (OUT_F32) {
#pragma unroll
          for (int n = 0; n < 2; ++n) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              *reinterpret_cast<f32x4*>(&os[ost_off(r, 2 * jj + h)]) =
                  (f32x4){O[n][4 * jj] * sc, O[n][4 * jj + 1] * sc, O[n][4 * jj + 2] * sc, O[n][4 * jj + 3] * sc};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int row = 8 * i + rr, col = 32 * n + 4 * cu;
              const u32x4 x = *reinterpret_cast<const u32x4*>(&os[ost_off(row, cu)]);
              buf_store_b128(x, ro, col < dv ? ((32 * W + row) * dv + col) * 4 : kOffOutOfRange);
            }
          }
        } else {
#pragma unroll
          for (int n = 0; n < 2; ++n)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              *reinterpret_cast<u32x2*>(&os[ost_off(r, 4 * n + jj) + 2 * h]) =
                  (u32x2){pack_bf16x2(O[n][4 * jj] * sc, O[n][4 * jj + 1] * sc),
                          pack_bf16x2(O[n][4 * jj + 2] * sc, O[n][4 * jj + 3] * sc)};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = 8 * i + rr, col = 8 * cu;
            const u32x4 x = *reinterpret_cast<const u32x4*>(&os[ost_off(row, cu)]);
            buf_store_b128(x, ro, col < dv ? ((32 * W + row) * dv + col) * 2 : kOffOutOfRange);
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
    update_blocks<NB>(L.KT, vtab(L, (c0 + c) & 1), S, ra, rb, r, h);
    if (GRAM) gram_update(L.KT, G, grow, h, 0, 1);
    // next chunk in registers (V with the current exponent), and the maxima that decide the
    // next exponent: |S| before this update, |v| and |k| of the next chunk
    stage_convert_qk<true>(st, cv, p.qs, p.ks, lane);
    stage_convert_v(st, cv);   // exponent 0; the rare path below converts again otherwise
    stage_pin<true>(cv);
    {
      const int par = (c + 1) & 1;
      const u32 mvk = wave_max_u16x2(more ? (stage_vmax(st) << 16) | stage_kmax(st) : 0u);
      if (lane == 0) {
        L.xs[par][W] = msS;
        L.xv[par][W] = mvk >> 16;
        L.xk[par][W] = mvk & 0xffffu;
      }
    }

    lds_barrier();   // every wave is done with this chunk's tables and the published state
    if (more) {
      stage_write<true>(cv, L.Q0, L.Kr, L.KT, vtab(L, (c0 + c + 1) & 1), lane, W);
      publish_state<NB>(L, S, OB::first, r, h);
      if (GRAM) publish_gram(L, G, r, h);
    }
    {
      // The state just published is below its max before this update plus a bound on this
      // chunk's increment, 128 max|k-side product| max|v 2^-U| (the table products are
      // (k~/2)^2-sized, k~/4 or 1/2); if that bound or the next chunk's V would leave fp16 the
      // exponent rises and the rare path rewrites what was just written (before the barrier).
      const int par = (c + 1) & 1;
      const int eS = exp_of_f32bits(lds_max4(L.xs[par]));
      const int eV = exp_of_f32bits(lds_max4(L.xv[par]) << 16);
      const int eK = exp_of_f32bits(lds_max4(L.xk[par]) << 16);
      const float kk = eKc == kNoExp ? 0.f : p.ks * __builtin_ldexpf(2.0f, eKc);
      const float kf = __builtin_fmaxf(kk * kk, __builtin_fmaxf(0.5f * kk, 0.5f));
      const float dS = eVc == kNoExp ? 0.f : 128.0f * kf * __builtin_ldexpf(2.0f, eVc - U);
      const float sb = (eS == kNoExp ? 0.f : __builtin_ldexpf(2.0f, eS)) + dS;
      const int Un = next_unit(U, exp_of_f32bits(__builtin_bit_cast(u32, sb)), eV);
      if (Un != U || (Un != 0 && more)) {   // rare, and the same in every wave
        if (Un != U) acc_scale<NB>(S, __builtin_ldexpf(1.0f, U - Un));
        if (more) {
          stage_convert_v_scaled(st, cv, __builtin_ldexpf(1.0f, -Un));
          stage_write_v(cv, vtab(L, (c0 + c + 1) & 1), lane, W);
          if (Un != U) publish_state<NB>(L, S, OB::first, r, h);
        }
        U = Un;
      }
      eVc = eV;
      eKc = eK;
    }
    if constexpr (LAYER) {
      if (W == 0 && lane == 0 && more) L.Us[(c0 + c + 1) & 1] = U;   // exponent of the next chunk's V^T
    }
    if (more) lds_barrier();
  }

  // ---- final state of the head (last segment) in the reference feature basis, fp32:
  // state_out[f][0..dv) = sum_u phi_f(k_u) v_u, state_out[f][dv] = sum_u phi_f(k_u)
  if (!LAYER && p.state_out != nullptr && (seg + 1) * p.ostride >= p.P) {
    float* so = p.state_out + (size_t)bh * 153 * (dv + 1);
    // the Gram matrix in fp32 for the k-sums: G32[i][j], 32 x 33 floats over the S^T table
    float* G32 = reinterpret_cast<float*>(L.ST);
    if (GRAM) {
#pragma unroll
      for (int e = 0; e < 16; ++e) G32[(8 * (e >> 2) + 4 * h + (e & 3)) * 33 + r] = G[e];
    }
    lds_barrier();
    const float su = __builtin_ldexpf(4.0f, U);   // state registers -> k side of 2p
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int blk = OB::first + b;
      // accumulator element e of lane half h is slot 32 blk + 16 (e >> 3) + 8 h + (e & 7)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int f = 32 * blk + 16 * (e >> 3) + 8 * h + (e & 7);
        const RefFeat rf = ref_feature(f);
        if (rf.ref < 0) continue;
        const float fac = p.st_fac[rf.fac] * su;
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
        const float z = 4.0f * fa * fb * G32[da * 33 + db];
        so[(size_t)rf.ref * (dv + 1) + dv] = rf.ref == 0 ? (float)N + p.prev_tokens : z * p.st_fac[rf.fac];
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

// Kernel 3 of the full layer: outputs of both branches, one work-group of 8 waves per (head,
// segment) (recurrence roles 0..3, softmax roles 4..7).
template <bool OUT_F32, int DSW>
__global__ __launch_bounds__(64 * 2 * NWAVE_OUT, 1) void chunked_layer_kernel(const ChunkParams p) {
  __shared__ __attribute__((aligned(16))) LayerLds<DSW> L;
  using LT = LayerLds<DSW>;
  int bh, seg;
  map_segment(blockIdx.x, p.BH, (p.P + p.ostride - 1) / p.ostride, bh, seg);
  switch (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) {
    case 0: output_wave<0, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    case 1: output_wave<1, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    case 2: output_wave<2, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    case 3: output_wave<3, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    case 4: output_wave<4, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    case 5: output_wave<5, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    case 6: output_wave<6, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
    default: output_wave<7, true, OUT_F32, LT, DSW>(L, p, bh, seg); break;
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

int chunked_chunk_tokens() { return CH; }

size_t chunked_workspace_bytes(int BH, int N, int d, int dv, int chunk) {
  if (chunk < 1) return (size_t)-1;
  if (d != 16 || dv > 64) return general_chunked_bytes(BH, N, d, dv, false);
  int P, seg_chunks;
  segment_split(BH, N, P, seg_chunks);
  // per (head, segment): fp16 S^T, fp32 Gram matrix, two exponents
  const size_t per = (size_t)64 * NF * 2 + (size_t)1024 * 4 + 2 * sizeof(int);
  return (size_t)BH * P * per + 256;
}

size_t chunked_scratch_bytes(int BH, int N, int d, int dv, bool with_state, bool in_f32) {
  if (d != 16 || dv > 64 || in_f32) return with_state ? (size_t)-1 : general_chunked_bytes(BH, N, d, dv, in_f32);
  int P, seg_chunks;
  segment_split(BH, N, P, seg_chunks);
  if (P == 1 && !with_state) return 0;
  return chunked_workspace_bytes(BH, N, d, dv, 1);
}

namespace {

// Parameters of the chunked kernels shared by the chunked call and the full layer; P, seg_chunks
// and the workspace pointers from the segment split.
ChunkParams chunk_params(const void* q, const void* k, const void* v, void* out, void* workspace, int BH, int N,
                         int dv, float scale) {
  ChunkParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.out = out;
  p.BH = BH;
  p.N = N;
  p.dv = dv;
  int P, seg_chunks;
  segment_split(BH, N, P, seg_chunks);
  p.P = P;
  p.seg_chunks = seg_chunks;
  p.ostride = 1;
  const size_t nslot = (size_t)BH * P;
  char* ws = static_cast<char*>(workspace);
  p.wsS = reinterpret_cast<uint16_t*>(ws);
  p.wsG = reinterpret_cast<float*>(ws + nslot * 64 * NF * 2);
  p.wsE = reinterpret_cast<int*>(ws + nslot * (64 * NF * 2 + 1024 * 4));
  p.wsEP = p.wsE + nslot;
  // q~ = sqrt(scale) q (q~.k~ = s); the K^T table rows hold k~/2
  const double rc = sqrt((double)scale);
  p.qs = (float)rc;
  p.ks = (float)(0.5 * rc);
  // k side of 2p -> reference features: constant 2, linear k~, square k~^2, pair k~ k~
  p.st_fac[0] = 0.5f;
  p.st_fac[1] = 1.0f;
  p.st_fac[2] = (float)(1.0 / sqrt(2.0));
  p.st_fac[3] = 1.0f;
  for (int i = 0; i < 4; ++i) p.st_inv[i] = (float)(1.0 / (double)p.st_fac[i]);
  return p;
}

// Kernels 1 and 2 (state increments of every segment but the last, their prefixes); the
// initial-state import before them when p.state_in is set.
int launch_increments(const ChunkParams& p, bool vec_v, hipStream_t stream) {
  if (p.state_in != nullptr) {
    hipLaunchKernelGGL(chunked_import_kernel, dim3((unsigned)p.BH), dim3(256), 0, stream, p);
    const int e = (int)hipGetLastError();
    if (e != 0) return e;
  }
  if (p.P > 1) {
    const dim3 grid((unsigned)((p.BH * (p.P - 1) + SEG_PER_WG - 1) / SEG_PER_WG));
    const dim3 block(64 * NWAVE_SEG * SEG_PER_WG);
    if (vec_v)
      hipLaunchKernelGGL(chunked_segment_kernel<true>, grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL(chunked_segment_kernel<false>, grid, block, 0, stream, p);
    int e = (int)hipGetLastError();
    if (e != 0) return e;
    const dim3 pgrid((unsigned)((64 * NF / 4 + 1024 / 2 + 255) / 256), (unsigned)p.BH);
    hipLaunchKernelGGL(chunked_prefix_kernel, pgrid, dim3(256), 0, stream, p);
    e = (int)hipGetLastError();
    if (e != 0) return e;
  }
  return 0;
}

}  // namespace

int launch_based_chunked(const ChunkedArgs& a, hipStream_t stream) {
  if (a.d != 16 || a.dv > 64 || a.in_f32) {
    // other head dims and fp32 inputs: segment states + outputs; no state export or import
    if (a.state_out != nullptr || a.state_in != nullptr) return LA_ERR_UNSUPPORTED_DIM;
    return launch_general_chunked(a, stream);
  }
  if ((reinterpret_cast<uintptr_t>(a.q) & 7) || (reinterpret_cast<uintptr_t>(a.k) & 7)) return LA_ERR_BAD_ALIGNMENT;
  ChunkParams p = chunk_params(a.q, a.k, a.v, a.out, a.workspace, a.BH, a.N, a.dv, a.scale);
  p.state_out = a.state_out;
  p.state_in = a.state_in;
  p.den_out = a.den_out;
  p.prev_tokens = (float)a.prev_tokens;
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  const bool vec_v = (a.dv % 8 == 0) && ((reinterpret_cast<uintptr_t>(a.v) & 15) == 0);
  p.vec_out = (a.dv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.out) & 15) == 0);
  const int e = launch_increments(p, vec_v, stream);
  if (e != 0) return e;
  const dim3 grid((unsigned)(a.BH * p.P));
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

bool layer_fused_shape(int d, int dv, int dsw, int window) {
  return d == 16 && dv % 8 == 0 && dv <= 64 && (dsw == 16 || dsw == 32 || dsw == 64) && window >= 1 && window <= 64;
}

int launch_based_layer(const LayerArgs& a, hipStream_t stream) {
  if (!layer_fused_shape(a.d, a.dv, a.dsw, a.window)) return LA_ERR_UNSUPPORTED_DIM;
  ChunkParams p = chunk_params(a.q, a.k, a.v, a.out, a.workspace, a.BH, a.N, a.dv, a.scale);
  p.eps = a.eps;
  p.normalize = 1;
  p.out_f32 = a.out_f32 ? 1 : 0;
  p.vec_out = 1;
  p.qsw = static_cast<const uint16_t*>(a.qsw);
  p.ksw = static_cast<const uint16_t*>(a.ksw);
  p.window = a.window;
  p.sw_log2 = (float)((double)a.scale_sw * 1.4426950408889634);
  const int e = launch_increments(p, true, stream);
  if (e != 0) return e;
  // one 8-wave work-group per CU: when the (head, segment) work-groups would need more than one
  // round of the CUs, each takes two consecutive segments from the first one's prefix (one round,
  // one fixed phase per work-group instead of two)
  if (p.P >= 2 && (long long)a.BH * p.P > device_cu_count()) p.ostride = 2;
  const dim3 grid((unsigned)(a.BH * ((p.P + p.ostride - 1) / p.ostride))), block(64 * 2 * NWAVE_OUT);
#define LA_LAYER(F32, D) hipLaunchKernelGGL((chunked_layer_kernel<F32, D>), grid, block, 0, stream, p)
  if (a.dsw == 16) {
    if (a.out_f32) LA_LAYER(true, 16); else LA_LAYER(false, 16);
  } else if (a.dsw == 32) {
    if (a.out_f32) LA_LAYER(true, 32); else LA_LAYER(false, 32);
  } else {
    if (a.out_f32) LA_LAYER(true, 64); else LA_LAYER(false, 64);
  }
#undef LA_LAYER
  return (int)hipGetLastError();
}

}  // namespace la
