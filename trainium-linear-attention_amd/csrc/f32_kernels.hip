// fp32-input kernels (gfx950 fp32 MFMA) for the parallel BASED path and the sliding-window
// softmax path.
//
// Same block structure as the bf16 kernels -- per query block, the causal (or windowed) key
// blocks stream through LDS, scores are computed transposed (S^T = K Q^T) so they feed the
// P.V MFMA without shuffles -- but every operand stays fp32 (v_mfma_f32_32x32x2_f32).  These
// serve fp32 callers such as the reference's own CPU-sized configuration, where bf16 rounding
// of P would not meet a 1e-4 tolerance.
//
//   BASED   (kernels/pytorch_attention.py:33-41): scores start from 1/c so b = q.k + 1/c,
//           p = 1 + (c^2/2)(b*b - 1/c^2) = 1 + s + s^2/2, causal mask, den = row sum of p.
//   SLIDING (benchmarks/sliding_attention_benchmark.py:32-56): online softmax of c*q.k over
//           keys t-W+1..t, running max/sum per query.
#include <float.h>

#include "../../include/based_la.h"
#include "la_common.hpp"
#include "la_internal.hpp"

namespace la {

namespace {

constexpr int BNF = 64;
constexpr int VROWF = BNF + 4;   // floats; 68 dwords -> 16-byte reads hit distinct banks

__device__ __forceinline__ f32x16 mfma32x32x2_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

struct F32Params {
  const float* q;
  const float* k;
  const float* v;
  void* out;
  float* den;
  const float* addend;   // sliding: optional fp32 addend of the output, or null
  float* part;           // BASED key split: partial numerators [BH][nslot][BM][dv], then row sums
                         // [BH][nslot][BM] (null: no split); or f32_x6_split_kernel's partials
  int BH, N, d, dv, nqb, window, nslot;
  int x6parts;           // f32_x6_split_kernel: parts per query block slot (0: not used)
  int vec;               // d % 4 == 0, dv % 4 == 0 and q, k, v 16-byte aligned: float4 loads
  int out_vec;           // out 16-byte (fp32) / 8-byte (bf16) aligned: 4-column stores
  float inv_c, inv_c2, fscale, eps, scale_log2;
  int normalize, out_f32;
  int xcd_cus;           // CUs per XCD (the work-group order of f32_x6_tiled_kernel)
};

// Key-split slot w of a head's nslot = nqb (nqb + 1): query block qb = the largest with
// qb (qb + 1) <= w, then key block c = w - qb (qb + 1) (the float estimate is corrected exactly).
__device__ __forceinline__ void split_slot(int wg, int nslot, int& bh, int& qb, int& c) {
  bh = wg / nslot;
  const int w = wg - bh * nslot;
  int r = (int)((__builtin_sqrtf(4.0f * (float)w + 1.0f) - 1.0f) * 0.5f);
  while ((r + 1) * (r + 2) <= w) ++r;
  while (r * (r + 1) > w) --r;
  qb = r;
  c = w - r * (r + 1);
}

// SPLIT = 2 (BASED, small grids): two groups of four waves take the same 128 queries and every
// other key block each, with a staging double buffer per group, and add their numerators and
// row sums through LDS at the end, which halves the serial chain of key blocks of a query block.
// PART (BASED, small grids): work-group (head, query block qb, c) takes key block c only
// (c = 0 .. 2 qb + 1) and writes its unnormalised numerators and row sums to p.part; a combine
// kernel adds the 2 qb + 2 partials of every query in a fixed order and normalises.  This spreads
// a query block's keys over 2 qb + 2 compute units instead of one.
template <int KS, int MT, bool SLIDING, int SPLIT = 1, bool PART = false>
__global__ __launch_bounds__(256 * SPLIT) void f32_attn_kernel(const F32Params p) {
  static_assert(SPLIT == 1 || (SPLIT == 2 && !SLIDING), "key split: BASED only");
  static_assert(!PART || (SPLIT == 1 && !SLIDING), "partial sums: BASED, one wave group");
  constexpr int DK = 16 * KS, DV = 32 * MT, BM = 128, HALF = DK / 2;
  constexpr int KROW = DK + 4;
  constexpr int KCH = BNF * DK / 4;              // float4 chunks in a K block
  constexpr int KPT = (KCH + 255) / 256;
  constexpr int VGR = (DV / 4) * (BNF / 4);
  constexpr int VPT = (VGR + 255) / 256;

  __shared__ __attribute__((aligned(16))) float Ks[SPLIT][2][BNF * KROW];
  __shared__ __attribute__((aligned(16))) float VTs[SPLIT][2][DV * VROWF];

  const int tid_all = threadIdx.x, tid = SPLIT == 2 ? tid_all & 255 : tid_all;   // thread within its group
  const int grp = SPLIT == 2 ? __builtin_amdgcn_readfirstlane(tid_all >> 8) : 0;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv, W = p.window;
  int bh, qb, pc = 0;
  if (PART) {
    split_slot(blockIdx.x, p.nslot, bh, qb, pc);
  } else {
    map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb);
  }
  const int q0 = qb * BM;
  const int jlo = PART ? pc : (SLIDING ? max(0, q0 - W + 1) / BNF : 0);
  const int jhi = PART ? pc : min((N - 1) / BNF, (q0 + BM - 1) / BNF);
  const size_t hrow = (size_t)bh * N;
  const float* __restrict__ qg = p.q + hrow * d;
  const float* __restrict__ kg = p.k + hrow * d;
  const float* __restrict__ vg = p.v + hrow * dv;
  const int wq0 = q0 + 32 * w;
  const bool wave_live = wq0 < N;
  const int query = wq0 + n;

  // lane group h holds d-elements [HALF*h, HALF*h + HALF) of its query row
  float qf[HALF];
  if (p.vec && HALF % 4 == 0) {
#pragma unroll
    for (int e = 0; e < HALF; e += 4) {
      const int col = HALF * h + e;
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (query < N && col < d) x = *reinterpret_cast<const f32x4*>(qg + (size_t)query * d + col);
#pragma unroll
      for (int i = 0; i < 4; ++i) qf[e + i] = x[i];
    }
  } else {
#pragma unroll
    for (int e = 0; e < HALF; ++e) {
      const int col = HALF * h + e;
      qf[e] = (query < N && col < d) ? qg[(size_t)query * d + col] : 0.f;
    }
  }

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = splat16(0.f);
  float rsum = 0.f;        // BASED: row sum of p; SLIDING: running softmax sum
  float mrun = -FLT_MAX;   // SLIDING: running max (log2 domain)

  f32x4 kr[KPT];
  f32x4 vr[VPT][4];
  auto load = [&](int row0) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int c = tid + 256 * r;
      const int key = c / (DK / 4), col = 4 * (c % (DK / 4));
      const int row = row0 + key;
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (c < KCH && row < N) {
        if (p.vec) {
          if (col < d) x = *reinterpret_cast<const f32x4*>(kg + (size_t)row * d + col);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = (col + e < d) ? kg[(size_t)row * d + col + e] : 0.f;
        }
      }
      kr[r] = x;
    }
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int g = tid + 256 * r;
      const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + 4 * kg4 + i;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (g < VGR && row < N) {
          if (p.vec) {
            if (4 * g4 < dv) x = *reinterpret_cast<const f32x4*>(vg + (size_t)row * dv + 4 * g4);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = (4 * g4 + e < dv) ? vg[(size_t)row * dv + 4 * g4 + e] : 0.f;
          }
        }
        vr[r][i] = x;
      }
    }
  };
  auto store = [&](int s) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int c = tid + 256 * r;
      if (c < KCH) {
        const int key = c / (DK / 4), col = 4 * (c % (DK / 4));
        *reinterpret_cast<f32x4*>(&Ks[grp][s][key * KROW + col]) = kr[r];
      }
    }
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int g = tid + 256 * r;
      if (g < VGR) {
        const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<f32x4*>(&VTs[grp][s][(4 * g4 + c) * VROWF + 4 * kg4]) =
              (f32x4){vr[r][0][c], vr[r][1][c], vr[r][2][c], vr[r][3][c]};
      }
    }
  };

  load((jlo + grp) * BNF);
  store(0);
  __syncthreads();
  const float inv_c = p.inv_c, inv_c2 = p.inv_c2, fscale = p.fscale, sl2 = p.scale_log2;

  // group grp takes key blocks jlo + grp, jlo + grp + SPLIT, ...; every thread runs the same
  // number of iterations (and barriers), a group past its last block idles in the last one
  const int niter = (jhi - jlo + SPLIT) / SPLIT;
  for (int it = 0; it < niter; ++it) {
    const int j = jlo + SPLIT * it + grp;
    const int s = it & 1;
    const bool more = SPLIT == 1 ? j < jhi : it + 1 < niter;
    if (more) load((j + SPLIT) * BNF);
    if (wave_live && (SPLIT == 1 || j <= jhi)) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int kb = j * BNF + 32 * ks;
        if (kb > wq0 + 31) continue;
        if (SLIDING && kb + 31 < wq0 - W + 1) continue;
        f32x16 b = splat16(SLIDING ? 0.f : inv_c);
        const float* kp = &Ks[grp][s][(32 * ks + n) * KROW + HALF * h];
#pragma unroll
        for (int e = 0; e < HALF; ++e) b = mfma32x32x2_f32(kp[e], qf[e], b);
        float pv[16];
        if (!SLIDING) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float u = __builtin_fmaf(b[i], b[i], -inv_c2);
            float pe = __builtin_fmaf(fscale, u, 1.0f);
            if (kb + c32_row(i, h) > query) pe = 0.f;
            pv[i] = pe;
            rsum += pe;
          }
        } else {
          float mloc = -FLT_MAX;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb + c32_row(i, h);
            const bool ok = key <= query && key >= query - W + 1;
            pv[i] = ok ? b[i] * sl2 : -FLT_MAX;
            mloc = fmaxf(mloc, pv[i]);
          }
          mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
          const float mnew = fmaxf(mrun, mloc);
          const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
          mrun = mnew;
          float l = rsum * alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float e = (pv[i] == -FLT_MAX) ? 0.f : __builtin_amdgcn_exp2f(pv[i] - mnew);
            pv[i] = e;
            l += e;
          }
          rsum = l;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][i] *= alpha;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 vv = *reinterpret_cast<const f32x4*>(&VTs[grp][s][(32 * mt + n) * VROWF + 32 * ks + 8 * g + 4 * h]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt] = mfma32x32x2_f32(vv[e], pv[4 * g + e], acc[mt]);
          }
        }
      }
    }
    if (more) store(s ^ 1);
    __syncthreads();
  }

  if (SPLIT == 2) {
    // group 1 hands its numerators and row sums to group 0 through the (now free) stages
    float* red = &VTs[0][0][0];
    static_assert(SPLIT == 1 || 4 * (MT * 16 + 1) * 64 <= SPLIT * 2 * DV * VROWF, "reduction fits");
    if (grp == 1 && wave_live) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[((w * MT + mt) * 16 + i) * 64 + lane] = acc[mt][i];
      red[(4 * MT * 16 + w) * 64 + lane] = rsum;
    }
    __syncthreads();
    if (grp == 1) return;
    if (wave_live) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][i] += red[((w * MT + mt) * 16 + i) * 64 + lane];
      rsum += red[(4 * MT * 16 + w) * 64 + lane];
    }
  }

  if (!wave_live) return;
  const float rs = rsum + __shfl_xor(rsum, 32);
  if (PART) {
    // slot (bh, qb, pc) in the accumulator order [wave][mt][lane][16] (DV = 32 MT columns), so
    // that every lane stores whole 16-byte pieces and the wave one contiguous run per mt
    const size_t slot = (size_t)bh * p.nslot + (size_t)qb * (qb + 1) + pc;
    float* num = p.part + (slot * 4 + w) * (size_t)(MT * 1024) + 16 * lane;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(num + mt * 1024 + 4 * g) =
            (f32x4){acc[mt][4 * g], acc[mt][4 * g + 1], acc[mt][4 * g + 2], acc[mt][4 * g + 3]};
    if (h == 0) p.part[(size_t)p.BH * p.nslot * 128 * (MT * 32) + slot * BM + 32 * w + n] = rs;
    return;
  }
  if (query >= N) return;
  float inv;
  if (SLIDING) {
    inv = 1.0f / rs;
  } else {
    inv = p.normalize ? 1.0f / (rs + p.eps) : 1.0f;
    if (p.den != nullptr && h == 0) p.den[hrow + query] = rs;
  }
  const size_t obase = (hrow + query) * (size_t)dv;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int col = 32 * mt + c32_row(i, h);
      if (col < dv) {
        float y = acc[mt][i] * inv;
        if (SLIDING && p.addend != nullptr) y += p.addend[obase + col];
        if (p.out_f32)
          static_cast<float*>(p.out)[obase + col] = y;
        else
          static_cast<uint16_t*>(p.out)[obase + col] = f32_to_bf16_bits(y);
      }
    }
}

// Combine of the key-split partials of query block qb: slots c = 0 .. 2 qb + 1 added in that
// order and normalised.  The numerators are in the split kernel's accumulator order
// [wave][mt][lane][16]: thread -> one 16-byte piece (wave w, mt, lane (n, h), group g), i.e. query
// 32 w + n, columns 32 mt + 8 g + 4 h .. +3, read coalesced from every slot; a batch of eight
// slots is loaded before any is added (a dependent load per slot would serialise on the L2
// latency).  Work-group (head, query block, 256 pieces).
template <int MT>
__global__ __launch_bounds__(256) void f32_split_combine_kernel(const F32Params p) {
  constexpr int BM = 128, PIECES = 4 * MT * 64 * 4, WPB = PIECES / 256;
  const int tid = threadIdx.x, bh = blockIdx.y, qb = blockIdx.x / WPB;
  const int pc = (blockIdx.x - qb * WPB) * 256 + tid;    // piece
  const int w = pc / (MT * 256), mt = (pc / 256) % MT, lane = (pc / 4) % 64, g = pc % 4;
  const int n = lane & 31, h = lane >> 5;
  const int N = p.N, dv = p.dv, q0 = qb * BM, row = q0 + 32 * w + n, col = 32 * mt + 8 * g + 4 * h;
  if (row >= N) return;
  const int ns = 2 * qb + 2;
  const size_t slot0 = (size_t)bh * p.nslot + (size_t)qb * (qb + 1);
  const float* dens = p.part + (size_t)p.BH * p.nslot * BM * (MT * 32);
  const float* base = p.part + slot0 * (size_t)(BM * MT * 32) + (size_t)w * (MT * 1024) + mt * 1024 + 16 * lane + 4 * g;
  float den = 0.f;
  f32x4 x = {0.f, 0.f, 0.f, 0.f};
  for (int b0 = 0; b0 < ns; b0 += 8) {
    float t[8];
    f32x4 u[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const bool ok = b0 + c < ns;
      t[c] = ok ? dens[(slot0 + b0 + c) * BM + 32 * w + n] : 0.f;
      u[c] = ok ? *reinterpret_cast<const f32x4*>(base + (size_t)(b0 + c) * (BM * MT * 32)) : (f32x4){0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      den += t[c];
      x += u[c];
    }
  }
  const size_t hrow = (size_t)bh * N;
  if (p.den != nullptr && col == 0) p.den[hrow + row] = den;
  const float inv = p.normalize ? 1.0f / (den + p.eps) : 1.0f;
  const size_t o = (hrow + row) * (size_t)dv + col;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (col + e >= dv) break;
    if (p.out_f32)
      static_cast<float*>(p.out)[o + e] = x[e] * inv;
    else
      static_cast<uint16_t*>(p.out)[o + e] = f32_to_bf16_bits(x[e] * inv);
  }
}

// fp32 BASED for small grids on bf16 MFMAs (d <= 16, dv <= 64, q / k / v rows 16-byte aligned).
// Every fp32 operand x is carried as three bf16 terms, x = x0 + x1 + x2 with x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1) (the differences are exact in fp32; the three terms
// hold x's 24-bit significand), and every product as the six bf16 MFMAs of term pairs (i, j)
// with i + j <= 2 (the dropped ones are below 2^-24 of the product), accumulated in fp32: the
// scores S^T = K Q^T (started from 1/c, as in f32_attn_kernel) and O^T = V^T P^T.  One 32x32x16
// bf16 MFMA does the work of eight 32x32x2 fp32 ones in half their cycles, so the six of a
// product cost 3/8 of the fp32 form, and no second pass adds partial sums.
//
// Work-group (head, 32 queries q0 .. q0 + 31), 8 waves: wave w takes the 32-key tiles u = w,
// w + 8, ... up to the queries' own (diagonal) tile.  Per tile it loads the K and V rows (fp32,
// 1 KB per load instruction) into registers one tile ahead, splits them and stores the three
// terms row-major in its own LDS region (16-byte chunks XOR-swizzled by row), reads the K
// fragments with ds_read_b128 and the V^T fragments with ds_read_b64_tr_b16 (as in the resident
// sliding-window kernel: the key order of a V^T fragment is the accumulator row order of the
// score tile, so P^T needs no shuffle).  At the end the waves' numerators and row sums are added
// through LDS in wave order (deterministic) and wave 0 normalises and stores.
struct Split3 {
  u32 t[3];
};
__device__ __forceinline__ Split3 split3_bf16x2(float a, float b) {
  Split3 r;
  r.t[0] = pack_bf16x2(a, b);
  const float ra = a - bf16_lo_to_f32(r.t[0]), rb = b - bf16_hi_to_f32(r.t[0]);
  r.t[1] = pack_bf16x2(ra, rb);
  r.t[2] = pack_bf16x2(ra - bf16_lo_to_f32(r.t[1]), rb - bf16_hi_to_f32(r.t[1]));
  return r;
}

// acc += A B over the term pairs (i, j), i + j <= 2, smallest first
__device__ __forceinline__ f32x16 mfma_split3(const u32x4 (&a)[3], const u32x4 (&b)[3], f32x16 acc) {
  acc = mfma32x32x16(a[1], b[1], acc);
  acc = mfma32x32x16(a[2], b[0], acc);
  acc = mfma32x32x16(a[0], b[2], acc);
  acc = mfma32x32x16(a[1], b[0], acc);
  acc = mfma32x32x16(a[0], b[1], acc);
  return mfma32x32x16(a[0], b[0], acc);
}

template <int MT>
__global__ __launch_bounds__(512) void f32_x6_kernel(const F32Params p) {
  constexpr int NW = 8, DV = 32 * MT, KT = 32;
  constexpr int VCH = DV / 8;                 // 16-byte chunks per V row (bf16)
  constexpr int VP = KT * DV / 4 / 64;        // f32x4 pieces of a V tile per lane
  typedef short v4s __attribute__((ext_vector_type(4)));
  // per wave and term: K rows [KT][16], then V rows [KT][DV] (bf16)
  constexpr int TAB = KT * 16 + KT * DV;
  __shared__ __attribute__((aligned(16))) uint16_t tabs[NW * 3 * TAB];
  static_assert(NW * 64 * (MT * 16 + 1) * 4 <= (int)sizeof(tabs), "reduction fits");

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, n = lane & 31, gh = (lane >> 4) & 1, gi = lane & 15;
  const int N = p.N, d = p.d, dv = p.dv;
  int bh, qb;
  map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb);
  const int q0 = KT * qb, query = q0 + n;
  const int ud = min(qb, (N - 1) / KT);   // the diagonal tile
  const size_t hrow = (size_t)bh * N;
  const float* __restrict__ qg = p.q + hrow * d;
  const float* __restrict__ kg = p.k + hrow * d;
  const float* __restrict__ vg = p.v + hrow * dv;
  uint16_t* const mine = tabs + 3 * w * TAB;
  // V row r keeps 16-byte chunk c at c ^ (4 bit1(r)) when it has 8 chunks: the transposed reads
  // of rows r .. r + 3 (four chunks each, 32 lanes per pass) then cover all 64 banks
  auto vswz = [](int r) { return VCH >= 8 ? ((r >> 1) & 1) << 2 : 0; };

  // Q^T fragment: lane (query n, half h) holds dims 8h .. 8h + 7, as three terms
  u32x4 qf[3];
  {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const int col = 8 * h + e;
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
      if (query < N && col < d) t = *reinterpret_cast<const f32x4*>(qg + (size_t)query * d + col);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[e + i] = t[i];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Split3 t = split3_bf16x2(x[2 * c], x[2 * c + 1]);
#pragma unroll
      for (int r = 0; r < 3; ++r) qf[r][c] = t.t[r];
    }
  }

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = splat16(0.f);
  float rsum = 0.f;

  // raw tile in registers: K piece i = key 16 i + lane / 4, dims 4 (lane % 4) .. +3; V piece i =
  // key (64 i + lane) / (DV / 4), columns 4 ((64 i + lane) % (DV / 4)) .. +3
  f32x4 kr[2], vr[VP];
  auto load = [&](int u) {
    const int kb = KT * u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = kb + 16 * i + (lane >> 2), col = 4 * (lane & 3);
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (key < N && col < d) x = *reinterpret_cast<const f32x4*>(kg + (size_t)key * d + col);
      kr[i] = x;
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      const int c = 64 * i + lane, key = kb + c / (DV / 4), col = 4 * (c % (DV / 4));
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (key < N && col < dv) x = *reinterpret_cast<const f32x4*>(vg + (size_t)key * dv + col);
      vr[i] = x;
    }
  };
  auto put = [&](int off, const f32x4& x) {
    const Split3 a = split3_bf16x2(x[0], x[1]), b = split3_bf16x2(x[2], x[3]);
#pragma unroll
    for (int r = 0; r < 3; ++r) *reinterpret_cast<u32x2*>(&mine[r * TAB + off]) = (u32x2){a.t[r], b.t[r]};
  };
  // K row r: 16-byte chunk c at position c ^ bit 4 of r (the fragment reads of rows n, chunk h
  // then fill all bank groups per pass); V rows: vswz
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = 16 * i + (lane >> 2), col4 = lane & 3;
      put(key * 16 + 8 * ((col4 >> 1) ^ ((key >> 4) & 1)) + 4 * (col4 & 1), kr[i]);
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      const int c = 64 * i + lane, key = c / (DV / 4), col4 = c % (DV / 4);
      put(KT * 16 + key * DV + 8 * ((col4 >> 1) ^ vswz(key)) + 4 * (col4 & 1), vr[i]);
    }
  };
  const float inv_c = p.inv_c, inv_c2 = p.inv_c2, fscale = p.fscale;
  auto tile = [&](int u) {
    const int kb = KT * u;
    u32x4 kf[3];
#pragma unroll
    for (int r = 0; r < 3; ++r)
      kf[r] = *reinterpret_cast<const u32x4*>(&mine[r * TAB + n * 16 + 8 * (h ^ ((n >> 4) & 1))]);
    const f32x16 b = mfma_split3(kf, qf, splat16(inv_c));
    // element i of lane (query n, half h) is key kb + c32_row(i, h)
    const bool interior = kb + KT - 1 <= q0 && kb + KT <= N;   // every key before every query
    float pr[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb + c32_row(i, h);
      const float uu = __builtin_fmaf(b[i], b[i], -inv_c2);
      const float pe = __builtin_fmaf(fscale, uu, 1.0f);
      pr[i] = (interior || (key <= query && key < N)) ? pe : 0.f;
      rsum += pr[i];
    }
    u32x4 pf[2][3];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Split3 s3 = split3_bf16x2(pr[8 * m + 2 * c], pr[8 * m + 2 * c + 1]);
#pragma unroll
        for (int r = 0; r < 3; ++r) pf[m][r][c] = s3.t[r];
      }
    // V^T fragment (m): keys 16 m + 8 (e / 4) + 4 h + e % 4 of element e, two transposed reads of
    // rows 16 m + 8 s2 + 4 h + 0..3 per term
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        u32x4 vf[3];
#pragma unroll
        for (int r = 0; r < 3; ++r) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int row = 16 * m + 8 * s2 + 4 * h + (gi >> 2);
            const int col = 32 * mt + 16 * gh + 4 * (gi & 3);
            const uint16_t* src = &mine[r * TAB + KT * 16 + row * DV + 8 * ((col >> 3) ^ vswz(row)) + (col & 7)];
            const v4s r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)src);
            const u32x2 r2 = __builtin_bit_cast(u32x2, r4);
            vf[r][2 * s2] = r2[0];
            vf[r][2 * s2 + 1] = r2[1];
          }
        }
        acc[mt] = mfma_split3(vf, pf[m], acc[mt]);
      }
  };

  if (w <= ud) load(w);
  for (int u = w; u <= ud; u += NW) {
    store();   // this wave's region; its reads of the previous tile were issued before (in order)
    if (u + NW <= ud) load(u + NW);
    tile(u);
  }

  // wave-ordered sum of the numerators and row sums (the tables are free after the barrier):
  // every active wave parks its partial numerators as MT * 4 slices of four columns per lane
  // and its row sums; wave s < 4 MT then adds slice s of all of them, in wave order, and stores
  // its four columns of the outputs
  constexpr int NSL = 4 * MT;
  const int nact = min(NW, ud + 1);
  float* red = reinterpret_cast<float*>(tabs);
  __syncthreads();
  if (w < nact) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(&red[((w * NSL + 4 * mt + g) * 64 + lane) * 4]) =
            (f32x4){acc[mt][4 * g], acc[mt][4 * g + 1], acc[mt][4 * g + 2], acc[mt][4 * g + 3]};
    red[NW * NSL * 256 + w * 64 + lane] = rsum;
  }
  __syncthreads();
  if (w >= NSL) return;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  float rs = 0.f;
  for (int ww = 0; ww < nact; ++ww) {
    y += *reinterpret_cast<const f32x4*>(&red[((ww * NSL + w) * 64 + lane) * 4]);
    rs += red[NW * NSL * 256 + ww * 64 + lane];
  }
  rs += __shfl_xor(rs, 32);
  if (query >= N) return;
  const float inv = p.normalize ? 1.0f / (rs + p.eps) : 1.0f;
  if (p.den != nullptr && w == 0 && h == 0) p.den[hrow + query] = rs;
  const size_t obase = (hrow + query) * (size_t)dv;
  const int col = 32 * (w >> 2) + 8 * (w & 3) + 4 * h;
  if (col < dv) {
    if (p.out_f32)
      *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + obase + col) = (f32x4){y[0] * inv, y[1] * inv, y[2] * inv, y[3] * inv};
    else
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + obase + col) =
          (u32x2){pack_bf16x2(y[0] * inv, y[1] * inv), pack_bf16x2(y[2] * inv, y[3] * inv)};
  }
}

// fp32 BASED on small grids with the keys split over work-groups (d <= 16, dv <= 64, 16-byte
// rows): the three-term bf16 products of f32_x6_kernel, but work-group (part, head, 32-query block
// qb) takes only key tiles 8 TPW part .. 8 TPW part + 8 TPW - 1 up to the diagonal one, TPW tiles
// per wave, so the longest serial chain is TPW tiles instead of ud / 8 + 1.  The operands go from
// global memory (L2) straight into MFMA registers, without LDS tables: lane (key n, half h) loads
// dims 8h .. 8h + 7 of its key for the score A operand, and element e of the V^T A operand of lane
// (column n, half h) is V[key 16 m + 8 (e / 4) + 4 h + e % 4][32 mt + n] (the score accumulator's
// row order), one coalesced 4-byte load per element.  The waves' numerators and row sums are added
// through LDS in wave order; a query block with a single part normalises and stores, the others
// write their partial numerators [query][DV] and row sums [query] to p.part for
// f32_x6_combine_kernel.
constexpr int X6_TPW = 2;   // key tiles per wave of f32_x6_split_kernel (1: 16.0, 2: 13.4, unsplit 14.6 us at B1 H4 N1024)
template <int MT>
__global__ __launch_bounds__(512, 2) void f32_x6_split_kernel(const F32Params p) {
  constexpr int NW = 8, DV = 32 * MT, KT = 32, NSL = 4 * MT, TP = NW * X6_TPW;
  __shared__ __attribute__((aligned(16))) float red[NW * NSL * 256 + NW * 64];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv, nqb = p.nqb;
  int g = blockIdx.x;
  const int qb = nqb - 1 - g % nqb;   // the heaviest query blocks first
  g /= nqb;
  const int bh = g % p.BH, part = g / p.BH;
  const int ud = min(qb, (N - 1) / KT);
  const int nparts = ud / TP + 1;
  if (part >= nparts) return;         // the whole work-group, before any barrier
  const int q0 = KT * qb, query = q0 + n;
  const size_t hrow = (size_t)bh * N;
  const float* __restrict__ qg = p.q + hrow * d;
  const float* __restrict__ kg = p.k + hrow * d;
  const float* __restrict__ vg = p.v + hrow * dv;

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = splat16(0.f);
  float rsum = 0.f;
  u32x4 qf[3];
  {
    float xq[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const int col = 8 * h + e;
      f32x4 tq = {0.f, 0.f, 0.f, 0.f};
      if (query < N && col < d) tq = *reinterpret_cast<const f32x4*>(qg + (size_t)query * d + col);
#pragma unroll
      for (int i = 0; i < 4; ++i) xq[e + i] = tq[i];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Split3 a = split3_bf16x2(xq[2 * c], xq[2 * c + 1]);
#pragma unroll
      for (int r = 0; r < 3; ++r) qf[r][c] = a.t[r];
    }
  }
  // every tile's loads first (the K rows, then the V elements), so that the second tile's data is
  // in flight during the first tile's products
  float xk[X6_TPW][8], xv[X6_TPW][MT][2][8];
#pragma unroll
  for (int j = 0; j < X6_TPW; ++j) {
    const int u = TP * part + w + NW * j;   // this wave's key tile
    const int kb = KT * u;
    const bool live = u <= ud;
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const int col = 8 * h + e;
      f32x4 tk = {0.f, 0.f, 0.f, 0.f};
      if (live && kb + n < N && col < d) tk = *reinterpret_cast<const f32x4*>(kg + (size_t)(kb + n) * d + col);
#pragma unroll
      for (int i = 0; i < 4; ++i) xk[j][e + i] = tk[i];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = kb + 16 * m + 8 * (e >> 2) + 4 * h + (e & 3), col = 32 * mt + n;
          xv[j][mt][m][e] = (live && key < N && col < dv) ? vg[(size_t)key * dv + col] : 0.f;
        }
  }
#pragma unroll
  for (int j = 0; j < X6_TPW; ++j) {
    const int u = TP * part + w + NW * j;
    if (u > ud) break;
    const int kb = KT * u;
    u32x4 kf[3];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Split3 b = split3_bf16x2(xk[j][2 * c], xk[j][2 * c + 1]);
#pragma unroll
      for (int r = 0; r < 3; ++r) kf[r][c] = b.t[r];
    }
    const f32x16 b = mfma_split3(kf, qf, splat16(p.inv_c));
    // element i of lane (query n, half h) is key kb + c32_row(i, h)
    const bool interior = kb + KT - 1 <= q0 && kb + KT <= N;
    float pr[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb + c32_row(i, h);
      const float pe = __builtin_fmaf(p.fscale, __builtin_fmaf(b[i], b[i], -p.inv_c2), 1.0f);
      pr[i] = (interior || (key <= query && key < N)) ? pe : 0.f;
      rsum += pr[i];
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      u32x4 pf[3];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Split3 s3 = split3_bf16x2(pr[8 * m + 2 * c], pr[8 * m + 2 * c + 1]);
#pragma unroll
        for (int r = 0; r < 3; ++r) pf[r][c] = s3.t[r];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 vf[3];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const Split3 s3 = split3_bf16x2(xv[j][mt][m][2 * c], xv[j][mt][m][2 * c + 1]);
#pragma unroll
          for (int r = 0; r < 3; ++r) vf[r][c] = s3.t[r];
        }
        acc[mt] = mfma_split3(vf, pf, acc[mt]);
      }
    }
  }

  // wave-ordered sum, as in f32_x6_kernel: wave s < 4 MT adds slice s (four columns per lane)
  const int nact = min(NW, ud + 1 - TP * part);
  if (w < nact) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int gg = 0; gg < 4; ++gg)
        *reinterpret_cast<f32x4*>(&red[((w * NSL + 4 * mt + gg) * 64 + lane) * 4]) =
            (f32x4){acc[mt][4 * gg], acc[mt][4 * gg + 1], acc[mt][4 * gg + 2], acc[mt][4 * gg + 3]};
    red[NW * NSL * 256 + w * 64 + lane] = rsum;
  }
  __syncthreads();
  if (w >= NSL) return;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  float rs = 0.f;
  for (int ww = 0; ww < nact; ++ww) {
    y += *reinterpret_cast<const f32x4*>(&red[((ww * NSL + w) * 64 + lane) * 4]);
    rs += red[NW * NSL * 256 + ww * 64 + lane];
  }
  rs += __shfl_xor(rs, 32);
  const int col = 32 * (w >> 2) + 8 * (w & 3) + 4 * h;
  if (nparts > 1) {
    const size_t slot = (size_t)(bh * nqb + qb) * p.x6parts + part;
    *reinterpret_cast<f32x4*>(p.part + slot * (KT * DV) + n * DV + col) = y;
    if (w == 0 && h == 0) p.part[(size_t)p.BH * nqb * p.x6parts * (KT * DV) + slot * KT + n] = rs;
    return;
  }
  if (query >= N) return;
  const float inv = p.normalize ? 1.0f / (rs + p.eps) : 1.0f;
  if (p.den != nullptr && w == 0 && h == 0) p.den[hrow + query] = rs;
  const size_t obase = (hrow + query) * (size_t)dv;
  if (col < dv) {
    if (p.out_f32)
      *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + obase + col) = (f32x4){y[0] * inv, y[1] * inv, y[2] * inv, y[3] * inv};
    else
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + obase + col) =
          (u32x2){pack_bf16x2(y[0] * inv, y[1] * inv), pack_bf16x2(y[2] * inv, y[3] * inv)};
  }
}

// The parts of f32_x6_split_kernel's query blocks with more than one: work-group (query block,
// head) adds the numerators and row sums of the parts in part order (all parts' loads issued
// before the first add), normalises and stores.
template <int MT>
__global__ __launch_bounds__(256) void f32_x6_combine_kernel(const F32Params p) {
  constexpr int KT = 32, DV = 32 * MT, PIECES = KT * DV / 4, NWP = 8;
  const int nqb = p.nqb, qb = blockIdx.x, bh = blockIdx.y, N = p.N, dv = p.dv;
  const int nparts = min(qb, (N - 1) / KT) / (8 * X6_TPW) + 1;
  if (nparts == 1) return;
  const size_t slot0 = (size_t)(bh * nqb + qb) * p.x6parts;
  const float* dens = p.part + (size_t)p.BH * nqb * p.x6parts * (KT * DV);
  const size_t hrow = (size_t)bh * N;
  for (int pc = threadIdx.x; pc < PIECES; pc += 256) {
    const int n = pc / (DV / 4), col = 4 * (pc % (DV / 4)), row = KT * qb + n;
    if (row >= N || col >= dv) continue;
    f32x4 x[NWP];
    float t[NWP];
#pragma unroll
    for (int c = 0; c < NWP; ++c) {
      const bool ok = c < nparts;
      x[c] = ok ? *reinterpret_cast<const f32x4*>(p.part + (slot0 + c) * (KT * DV) + n * DV + col)
                : (f32x4){0.f, 0.f, 0.f, 0.f};
      t[c] = ok ? dens[(slot0 + c) * KT + n] : 0.f;
    }
    f32x4 y = x[0];
    float den = t[0];
#pragma unroll
    for (int c = 1; c < NWP; ++c) {
      y += x[c];
      den += t[c];
    }
    if (p.den != nullptr && col == 0) p.den[hrow + row] = den;
    const float inv = p.normalize ? 1.0f / (den + p.eps) : 1.0f;
    const size_t o = (hrow + row) * (size_t)dv + col;
    if (p.out_f32)
      *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + o) = (f32x4){y[0] * inv, y[1] * inv, y[2] * inv, y[3] * inv};
    else
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + o) =
          (u32x2){pack_bf16x2(y[0] * inv, y[1] * inv), pack_bf16x2(y[2] * inv, y[3] * inv)};
  }
}

// fp32 BASED on larger grids, with the three-term bf16 products of f32_x6_kernel: work-group
// (head, 128 queries), wave w owns queries q0 + 32 w .. +31 and all DV columns.  The 32-key
// tiles of K and V pass through LDS once per work-group as their three bf16 terms (K rows
// [3][32][16], V rows [3][32][DV], double-buffered): each thread loads one K piece and DV / 32
// V pieces of the next tile into registers while the current one is computed, then splits and
// stores them behind one barrier per tile.  Scores, the causal mask, p, its split and
// O^T += V^T P^T are as in f32_x6_kernel; every wave finishes its own queries (no reduction).
template <int MT, int NW>
__global__ __launch_bounds__(64 * NW) void f32_x6_tiled_kernel(const F32Params p) {
  constexpr int DV = 32 * MT, KT = 32, BM = 32 * NW, NT = 64 * NW;
  constexpr int VCH = DV / 8;
  constexpr int VP = (KT * DV / 4 + NT - 1) / NT;   // V float4 pieces of a tile per thread
  typedef short v4s __attribute__((ext_vector_type(4)));
  constexpr int TAB = KT * 16 + KT * DV;      // halves per term: K rows, then V rows
  __shared__ __attribute__((aligned(16))) uint16_t tabs[2][3 * TAB];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, n = lane & 31, gh = (lane >> 4) & 1, gi = lane & 15;
  const int N = p.N, d = p.d, dv = p.dv;
  int bh, qb;
  // two work-groups per CU at dv > 32: the first round paired by size (B2 H16 N8192 902.9 ->
  // 866.5 us, B2 H16 N4096 285.9 -> 272.6 us in one process)
  map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb, MT == 2 ? p.xcd_cus : 0);
  const int q0 = BM * qb, wq0 = q0 + 32 * w, query = wq0 + n;
  const bool wave_live = wq0 < N;
  const int ud = min((q0 + BM - 1) / KT, (N - 1) / KT);   // last tile with a key <= a query
  const size_t hrow = (size_t)bh * N;
  const float* __restrict__ qg = p.q + hrow * d;
  const float* __restrict__ kg = p.k + hrow * d;
  const float* __restrict__ vg = p.v + hrow * dv;
  auto vswz = [](int r) { return VCH >= 8 ? ((r >> 1) & 1) << 2 : 0; };

  u32x4 qf[3];
  {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const int col = 8 * h + e;
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
      if (query < N && col < d) t = *reinterpret_cast<const f32x4*>(qg + (size_t)query * d + col);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[e + i] = t[i];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Split3 t = split3_bf16x2(x[2 * c], x[2 * c + 1]);
#pragma unroll
      for (int r = 0; r < 3; ++r) qf[r][c] = t.t[r];
    }
  }
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = splat16(0.f);
  float rsum = 0.f;

  // next tile in registers: K piece = key tid / 4, dims 4 (tid % 4) (threads < 128); V piece i =
  // key (tid + NT i) / (DV / 4), columns 4 ((tid + NT i) % (DV / 4))
  f32x4 kr, vr[VP];
  auto load = [&](int u) {
    const int kb = KT * u;
    {
      const int key = kb + (tid >> 2), col = 4 * (tid & 3);
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (tid < 128 && key < N && col < d) x = *reinterpret_cast<const f32x4*>(kg + (size_t)key * d + col);
      kr = x;
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      const int c = tid + NT * i, key = kb + c / (DV / 4), col = 4 * (c % (DV / 4));
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (c < KT * DV / 4 && key < N && col < dv) x = *reinterpret_cast<const f32x4*>(vg + (size_t)key * dv + col);
      vr[i] = x;
    }
  };
  auto put = [&](uint16_t* t3, int off, const f32x4& x) {
    const Split3 a = split3_bf16x2(x[0], x[1]), b = split3_bf16x2(x[2], x[3]);
#pragma unroll
    for (int r = 0; r < 3; ++r) *reinterpret_cast<u32x2*>(&t3[r * TAB + off]) = (u32x2){a.t[r], b.t[r]};
  };
  auto store = [&](int buf) {
    uint16_t* t3 = tabs[buf];
    if (tid < 128) {
      const int key = tid >> 2, col4 = tid & 3;
      put(t3, key * 16 + 8 * ((col4 >> 1) ^ ((key >> 4) & 1)) + 4 * (col4 & 1), kr);
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      const int c = tid + NT * i, key = c / (DV / 4), col4 = c % (DV / 4);
      if (c < KT * DV / 4) put(t3, KT * 16 + key * DV + 8 * ((col4 >> 1) ^ vswz(key)) + 4 * (col4 & 1), vr[i]);
    }
  };
  const float inv_c = p.inv_c, inv_c2 = p.inv_c2, fscale = p.fscale;
  auto tile = [&](int buf, int u) {
    const uint16_t* t3 = tabs[buf];
    const int kb = KT * u;
    u32x4 kf[3];
#pragma unroll
    for (int r = 0; r < 3; ++r)
      kf[r] = *reinterpret_cast<const u32x4*>(&t3[r * TAB + n * 16 + 8 * (h ^ ((n >> 4) & 1))]);
    const f32x16 b = mfma_split3(kf, qf, splat16(inv_c));
    const bool interior = kb + KT - 1 <= wq0 && kb + KT <= N;
    float pr[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb + c32_row(i, h);
      const float uu = __builtin_fmaf(b[i], b[i], -inv_c2);
      const float pe = __builtin_fmaf(fscale, uu, 1.0f);
      pr[i] = (interior || (key <= query && key < N)) ? pe : 0.f;
      rsum += pr[i];
    }
    u32x4 pf[2][3];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Split3 s3 = split3_bf16x2(pr[8 * m + 2 * c], pr[8 * m + 2 * c + 1]);
#pragma unroll
        for (int r = 0; r < 3; ++r) pf[m][r][c] = s3.t[r];
      }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        u32x4 vf[3];
#pragma unroll
        for (int r = 0; r < 3; ++r) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int row = 16 * m + 8 * s2 + 4 * h + (gi >> 2);
            const int col = 32 * mt + 16 * gh + 4 * (gi & 3);
            const uint16_t* src = &t3[r * TAB + KT * 16 + row * DV + 8 * ((col >> 3) ^ vswz(row)) + (col & 7)];
            const v4s r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)src);
            const u32x2 r2 = __builtin_bit_cast(u32x2, r4);
            vf[r][2 * s2] = r2[0];
            vf[r][2 * s2 + 1] = r2[1];
          }
        }
        acc[mt] = mfma_split3(vf, pf[m], acc[mt]);
      }
  };

  load(0);
  store(0);
  __syncthreads();
  for (int u = 0; u <= ud; ++u) {
    if (u < ud) load(u + 1);
    if (wave_live && KT * u <= wq0 + 31) tile(u & 1, u);
    if (u < ud) store((u + 1) & 1);
    __syncthreads();
  }

  if (!wave_live || query >= N) return;
  const float rs = rsum + __shfl_xor(rsum, 32);
  const float inv = p.normalize ? 1.0f / (rs + p.eps) : 1.0f;
  if (p.den != nullptr && h == 0) p.den[hrow + query] = rs;
  const size_t obase = (hrow + query) * (size_t)dv;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = 32 * mt + 8 * g + 4 * h;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = acc[mt][4 * g + e] * inv;
      if (col < dv) {
        if (p.out_f32)
          *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + obase + col) = (f32x4){y[0], y[1], y[2], y[3]};
        else
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + obase + col) =
              (u32x2){pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      }
    }
}

template <int KS, int MT, bool SL>
int launch_f32(F32Params p, hipStream_t stream) {
  p.nqb = (p.N + 127) / 128;
  const dim3 grid((unsigned)(p.nqb * p.BH));
  if constexpr (!SL && KS == 1 && MT <= 2) {
    // d <= 16, dv <= 64 and 16-byte rows: three-term bf16 products.  Grids of 256-query blocks
    // that fill every CU twice share each key tile among 8 waves (f32_x6_tiled_kernel); others
    // run 32-query work-groups with the keys spread over 8 waves (f32_x6_kernel).
    if (p.vec && p.out_vec) {
      if ((long long)((p.N + 255) / 256) * p.BH >= 2LL * device_cu_count()) {
        p.nqb = (p.N + 255) / 256;
        hipLaunchKernelGGL((f32_x6_tiled_kernel<MT, 8>), dim3((unsigned)(p.nqb * p.BH)), dim3(512), 0, stream, p);
      } else if (p.x6parts > 0) {
        // query blocks of more than 8 key tiles: keys split over work-groups, then the combine
        p.nqb = (p.N + 31) / 32;
        hipLaunchKernelGGL(f32_x6_split_kernel<MT>, dim3((unsigned)(p.nqb * p.BH * p.x6parts)), dim3(512), 0, stream,
                           p);
        const int e = (int)hipGetLastError();
        if (e != 0) return e;
        hipLaunchKernelGGL(f32_x6_combine_kernel<MT>, dim3((unsigned)p.nqb, (unsigned)p.BH), dim3(256), 0, stream, p);
      } else {
        p.nqb = (p.N + 31) / 32;
        hipLaunchKernelGGL(f32_x6_kernel<MT>, dim3((unsigned)(p.nqb * p.BH)), dim3(512), 0, stream, p);
      }
      return (int)hipGetLastError();
    }
  }
  if constexpr (!SL) {
    if (p.part != nullptr && p.nslot > 0) {
      // key split over work-groups (the workspace was sized for it: f32_split_slots)
      hipLaunchKernelGGL((f32_attn_kernel<KS, MT, SL, 1, true>), dim3((unsigned)(p.BH * p.nslot)), dim3(256), 0,
                         stream, p);
      hipLaunchKernelGGL(f32_split_combine_kernel<MT>, dim3((unsigned)(p.nqb * 4 * MT), (unsigned)p.BH), dim3(256), 0,
                         stream, p);
      return (int)hipGetLastError();
    }
  }
  if constexpr (!SL && KS == 1 && MT <= 2) {
    // fewer query blocks than CUs: split every query block's keys over two wave groups
    if ((long long)p.nqb * p.BH < device_cu_count()) {
      hipLaunchKernelGGL((f32_attn_kernel<KS, MT, SL, 2>), grid, dim3(512), 0, stream, p);
      return (int)hipGetLastError();
    }
  }
  hipLaunchKernelGGL((f32_attn_kernel<KS, MT, SL>), grid, dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

template <int KS, bool SL>
int dispatch_f32_mt(const F32Params& p, hipStream_t stream) {
  if (p.dv <= 32) return launch_f32<KS, 1, SL>(p, stream);
  if (p.dv <= 64) return launch_f32<KS, 2, SL>(p, stream);
  return launch_f32<KS, 4, SL>(p, stream);
}

template <bool SL>
int dispatch_f32(const F32Params& p, hipStream_t stream) {
  if (p.d <= 16) return dispatch_f32_mt<1, SL>(p, stream);
  if (p.d <= 32) return dispatch_f32_mt<2, SL>(p, stream);
  if (p.d <= 64) return dispatch_f32_mt<4, SL>(p, stream);
  return dispatch_f32_mt<8, SL>(p, stream);
}

}  // namespace

// Key split of the fp32 BASED kernel: for grids of fewer 128-query blocks than 256 (a quarter of
// MI355X's work-group slots) with at least two query blocks, every (query block, 64-key block)
// runs as its own work-group.  Slots per head (2 qb + 2 for query block qb), or 0 when the split
// is not used (also when its partials would pass 2048 slots in all).
int f32_split_slots(int BH, int N) {
  const long long nqb = (N + 127) / 128;
  if (nqb < 2 || nqb * BH >= 256) return 0;
  const long long ns = nqb * (nqb + 1);
  return ns * BH <= 2048 ? (int)ns : 0;
}

// Parts per query block of f32_x6_split_kernel (8 key tiles of 32 each), or 0 when it is not
// used: d > 16 or dv > 64, grids that f32_x6_tiled_kernel takes, and query blocks of at most 8
// tiles (N <= 256) or more than 64 (N > 2048, where the partials would outweigh the gain).
int f32_x6_split_parts(int BH, int N, int d, int dv) {
  if (d > 16 || dv > 64 || BH < 1 || N < 1) return 0;
  if ((long long)((N + 255) / 256) * BH >= 2LL * device_cu_count()) return 0;
  const int pm = ((N + 31) / 32 + 8 * X6_TPW - 1) / (8 * X6_TPW);
  return pm >= 2 && pm <= 8 ? pm : 0;
}

size_t f32_split_workspace_bytes(int BH, int N, int d, int dv) {
  const int ns = f32_split_slots(BH, N);
  const size_t cols = dv <= 32 ? 32 : (dv <= 64 ? 64 : 128);   // the kernel's 32 MT columns
  const size_t old = ns == 0 ? 0 : (size_t)BH * ns * 128 * (cols + 1) * sizeof(float);
  const int xp = f32_x6_split_parts(BH, N, d, dv);
  const size_t x6 = xp == 0 ? 0 : (size_t)BH * ((N + 31) / 32) * xp * 32 * (cols + 1) * sizeof(float);
  return old > x6 ? old : x6;
}

int launch_based_parallel_fp32(const ParallelArgs& a, hipStream_t stream) {
  F32Params p{};
  p.q = static_cast<const float*>(a.q);
  p.k = static_cast<const float*>(a.k);
  p.v = static_cast<const float*>(a.v);
  p.out = a.out;
  p.den = a.den;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  p.xcd_cus = device_cu_count() / 8;
  const float icf = (float)(1.0 / (double)a.scale);
  p.inv_c = icf;
  p.inv_c2 = (float)((double)icf * (double)icf);
  p.fscale = (float)(1.0 / (2.0 * (double)icf * (double)icf));
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  p.vec = (a.d % 4 == 0) && (a.dv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
          ((reinterpret_cast<uintptr_t>(a.k) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.v) & 15) == 0);
  p.out_vec = (reinterpret_cast<uintptr_t>(a.out) & (a.out_f32 ? 15 : 7)) == 0;
  p.nslot = f32_split_slots(a.BH, a.N);
  p.x6parts = (p.vec && p.out_vec) ? f32_x6_split_parts(a.BH, a.N, a.d, a.dv) : 0;
  if (p.nslot > 0 || p.x6parts > 0) {
    if (a.workspace == nullptr || a.workspace_bytes < f32_split_workspace_bytes(a.BH, a.N, a.d, a.dv))
      return LA_ERR_WORKSPACE;
    p.part = static_cast<float*>(a.workspace);
  }
  return dispatch_f32<false>(p, stream);
}

int launch_sliding_window_f32(const SlidingArgs& a, hipStream_t stream) {
  F32Params p{};
  p.q = static_cast<const float*>(a.q);
  p.k = static_cast<const float*>(a.k);
  p.v = static_cast<const float*>(a.v);
  p.out = a.out;
  p.addend = a.addend;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  p.window = a.window;
  p.scale_log2 = (float)((double)a.scale * 1.4426950408889634);
  p.out_f32 = a.out_f32 ? 1 : 0;
  p.vec = (a.d % 4 == 0) && (a.dv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
          ((reinterpret_cast<uintptr_t>(a.k) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.v) & 15) == 0);
  return dispatch_f32<true>(p, stream);
}

}  // namespace la
